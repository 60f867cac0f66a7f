/* nda_device.h - device helpers shared by the gfx950 kernels. */
#pragma once

#include "nda_internal.h"

namespace nda {

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoid_dev(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Which positions a row sees (the dispatch arithmetic of attention(),
// engine/src/nd_model.c:2451-2483), split into the shared-prefix run and
// the sequence's own slots. Own slots [0, n_own) are contiguous: without a
// shared prefix they are the sinks [0, n_sink) followed by the ring
// [n_sink, n_sink + rcount); with one they are ring indices [0, rcount).
struct Visible {
    int n_sh, n_own;
};

__device__ __forceinline__ Visible visible(const SeqDev &s, int p, int window)
{
    int sinks = min(s.n_sink, p + 1);
    int rcap = window - s.n_sink;
    int rcount = (p + 1 <= s.n_sink) ? 0 : min(p + 1 - s.n_sink, rcap);
    Visible v;
    v.n_sh = s.prefix >= 0 ? sinks : 0;
    v.n_own = s.prefix >= 0 ? rcount : sinks + rcount;
    return v;
}

// Own slot of position p (kv_slot, engine/src/nd_model.c:1302-1309, with the
// sinks of a shared prefix living outside the sequence's pages).
__device__ __forceinline__ int own_slot(const SeqDev &s, int p, int window)
{
    if (s.prefix >= 0)
        return (p - s.n_sink) % (window - s.n_sink);
    if (p < s.n_sink)
        return p;
    return s.n_sink + (p - s.n_sink) % (window - s.n_sink);
}

// v of lane (lane ^ M) of the wave, on VALU cross-lane operations rather
// than through the LDS crossbar (ds_bpermute): DPP within each 16-lane row
// (quad permutes for 1 and 2, the row shifted by 4 either way for 4, the row
// rotated by 8 for 8), row swaps for 16 and 32 (each returns (own, partner)
// in the lanes whose bit M is clear, (partner, own) in the others).
template <int M>
__device__ __forceinline__ float xor_lanes(float v, int lane)
{
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane distance");
    const int x = __builtin_bit_cast(int, v);
    int r;
    if constexpr (M == 1) {
        r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true);    // quad_perm [1, 0, 3, 2]
    } else if constexpr (M == 2) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true);    // quad_perm [2, 3, 0, 1]
    } else if constexpr (M == 4) {
        const int dn = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);   // row_shr:4, lane - 4
        const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, true);   // row_shl:4, lane + 4
        r = (lane & 4) ? dn : up;
    } else if constexpr (M == 8) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, true);   // row_ror:8
    } else if constexpr (M == 16) {
        const auto sw = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        r = (lane & 16) ? (int)sw[0] : (int)sw[1];
    } else {
        const auto sw = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        r = (lane & 32) ? (int)sw[0] : (int)sw[1];
    }
    return __builtin_bit_cast(float, r);
}

__device__ __forceinline__ int lane_id()
{
    return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ __forceinline__ float wave_max(float x)
{
    const int lane = lane_id();
    x = fmaxf(x, xor_lanes<32>(x, lane));
    x = fmaxf(x, xor_lanes<16>(x, lane));
    x = fmaxf(x, xor_lanes<8>(x, lane));
    x = fmaxf(x, xor_lanes<4>(x, lane));
    x = fmaxf(x, xor_lanes<2>(x, lane));
    return fmaxf(x, xor_lanes<1>(x, lane));
}

// One wave per (row, kv-head), lane = element. INT8: absmax over the row,
// scale = absmax/127 (1 for a zero row), then the engine's store
// (engine/src/nd_model.c:2426-2449 and kv_store_int8 :1819-1866) step for
// step: r = 1/scale, y = x*r, e = fma(-scale, y, x), q = fma(e, r, y) (a plain
// divide for |x| >= 1e30), clamp +-127, round half-to-even; a NaN quotient
// (scale below 2^-127, where 1/scale overflows) stores 0 as the host build
// does. F16: round to nearest even.
__device__ __forceinline__ int8_t quant_code(float x, float scale, float r)
{
    float q;
    if (x > -1e30f && x < 1e30f) {
        const float y = x * r;
        const float e = __builtin_fmaf(-scale, y, x);
        q = __builtin_fmaf(e, r, y);
    } else {
        q = __fdiv_rn(x, scale);
    }
    if (q != q)
        return 0;
    q = q > 127.0f ? 127.0f : q;
    q = q < -127.0f ? -127.0f : q;
    return (int8_t)(int)__builtin_rintf(q);
}

// Store one row of K and V (lane = element) for slot `off` of a page's
// kv-head block at hb, whose rows are dk and dv elements long. Shared by the
// append kernel, the fused append of the decode kernel and the front.
template <int ES>
__device__ __forceinline__ void store_row(uint8_t *hb, int off, int P, float kx, float vx, int lane, int dk,
                                          int dv)
{
    if constexpr (ES == 2) {
        if (lane < dk)
            reinterpret_cast<_Float16 *>(hb + (uint64_t)off * dk * 2)[lane] = (_Float16)kx;
        if (lane < dv)
            reinterpret_cast<_Float16 *>(hb + (uint64_t)P * dk * 2 + (uint64_t)off * dv * 2)[lane] = (_Float16)vx;
    } else {
        const float ak = wave_max(fabsf(kx)), av = wave_max(fabsf(vx));
        const float sk = ak > 0.0f ? __fdiv_rn(ak, 127.0f) : 1.0f;
        const float sv = av > 0.0f ? __fdiv_rn(av, 127.0f) : 1.0f;
        const float rk = __fdiv_rn(1.0f, sk), rv = __fdiv_rn(1.0f, sv);
        if (lane < dk)
            reinterpret_cast<int8_t *>(hb + (uint64_t)off * dk)[lane] = quant_code(kx, sk, rk);
        if (lane < dv)
            reinterpret_cast<int8_t *>(hb + (uint64_t)P * dk + (uint64_t)off * dv)[lane] = quant_code(vx, sv, rv);
        if (lane == 0) {
            float *sc = reinterpret_cast<float *>(hb + (uint64_t)P * (dk + dv));
            sc[off] = sk;
            sc[P + off] = sv;
        }
    }
}

} // namespace nda
