// nda_prefill.hip - causal prefill attention on MFMA (gfx950).
//
// The engine prefills one token at a time (esp32/main/main.c:233-234,
// :312-315): token t of a chunk attends every stored position <= pos + t. Over
// a chunk that is causal attention of n query tokens against pos + n keys, a
// dense contraction wherever a key tile lies below the earliest query of a
// row tile; only tiles that cross the diagonal are masked, tiles above it are
// never visited.
//
// A work-group owns 32*W query rows of one (sequence, kv-head); a row is one
// (token, query head of the group) pair, so GQA heads share every K/V tile.
// Key tiles of 32 are staged through LDS (K row-major, V transposed), then per
// wave and tile:
//   S^T[32 keys x 32 rows]  = K . Q^T           v_mfma_f32_32x32x16_f16
//   O^T[64 dims x 32 rows] += V^T . P^T         v_mfma_f32_32x32x16_f16
// Computing the transposes puts one query row in each lane (lane l and l+32
// hold halves of the keys), so the online-softmax state of a row is lane
// local, and the S^T accumulator registers are, slot for slot, the P^T
// operand of the next MFMA. Q and P are carried as fp16 hi + lo pairs (two
// MFMAs each) so the result keeps fp32-level accuracy: fp16 alone would leave
// ~2^-12 relative error on a dominant softmax weight.
//
// K/V are the cache's own fp16 values, or int8 codes (exact in fp16) with the
// per-(slot, kv-head) scales applied to S (k scale) and folded into P (v
// scale), the engine's dequantisation (engine/src/nd_model.c:2179-2180,
// :2250-2252).
#include "nda_device.h"

#include <float.h>

namespace nda {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int PF_KT = 32;   // keys per tile

__device__ __forceinline__ float max3(float a, float b, float c)
{
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

__device__ __forceinline__ float16v mfma32(half8 a, half8 b, float16v c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));

template <int ES, int DK, int DV, int NTHR>
struct PfTile {
    static constexpr int KPAD = DK + 8;        // halves per K row in LDS
    static constexpr int VPAD = PF_KT + 4;     // halves per V^T row in LDS
    static constexpr int KC = DK * ES / 16;    // 16-byte chunks per stored K row
    static constexpr int VC = DV * ES / 16;
    static constexpr int EPC = 16 / ES;        // elements per chunk
    static constexpr int NCHUNK = PF_KT * (KC + VC);
    static constexpr int CPT = (NCHUNK + NTHR - 1) / NTHR;   // chunks per thread
    static_assert(DK * ES % 16 == 0 && DV * ES % 16 == 0, "rows are whole 16-byte chunks");
};

// One thread's share of a K/V tile in flight: raw 16-byte chunks + scales.
template <int CPT>
struct Staged {
    u32x4 w[CPT];
    float sc[CPT];
};

// Element i of a dword as a half: fp16 lane or an int8 code (exact in fp16).
template <int ES>
__device__ __forceinline__ _Float16 code_at(uint32_t w, int i)
{
    if constexpr (ES == 1)
        return (_Float16)(float)(int8_t)(w >> (8 * i));
    else
        return __builtin_bit_cast(_Float16, (uint16_t)(w >> (16 * i)));
}

template <int ES, int DK, int DV, int REP, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W >= 8 ? 4 : 1)))
void prefill_kernel(PrefillArgs a)
{
    using T = PfTile<ES, DK, DV, 64 * W>;
    static_assert(DK % 16 == 0 && DV == 64, "prefill tiles: dk multiple of 16, dv 64");
    constexpr int ROWS = 32 * W;
    constexpr int NKB = DK / 16;               // k-blocks of the QK MFMA
    constexpr int NTHR = 64 * W;

    // two tile buffers: one is computed on while the next tile is written
    __shared__ __attribute__((aligned(16))) _Float16 Ks2[2][PF_KT][T::KPAD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt2[2][DV][T::VPAD];
    __shared__ float Ksc2[2][PF_KT], Vsc2[2][PF_KT];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int jh = lane >> 5, ln = lane & 31;
    // XCD-aware order: work-group w runs on XCD w % 8, so consecutive work
    // items (the row tiles of one sequence and kv-head, which read the same
    // K/V) are given to work-groups of one XCD and share its L2.
    const uint32_t nwg = gridDim.x, wg = blockIdx.x;
    const uint32_t item = (wg % 8u) * (nwg / 8u) + wg / 8u;
    const uint32_t b = a.items[3 * item];
    if (b == 0xFFFFFFFFu)
        return;
    const uint32_t g = a.items[3 * item + 1], rtile = a.items[3 * item + 2];
    const uint32_t seq = a.bseq[b];
    const SeqDev sd = a.seqs[seq];
    const int ntok = (int)a.bntok[b];
    const int nrows = ntok * REP;
    const int r0 = (int)rtile * ROWS;
    const int pos = sd.pos;
    const Visible vis0 = visible(sd, pos, (int)a.pg.window);
    const int n_sh = vis0.n_sh;                 // shared-prefix keys (fixed over the chunk)

    // this lane's query row
    const int r = r0 + wave * 32 + ln;
    const bool rvalid = r < nrows;
    const int tok = rvalid ? r / REP : 0;
    const int h = (int)g * REP + (rvalid ? r % REP : 0);
    const int qpos = pos + tok;                 // keys [0, qpos] visible
    const uint64_t qrow = (uint64_t)(a.btok0[b] + tok) * a.nh + h;

    // Q^T operand, hi and lo halves, slots = dims 16*kb + 8*jh + s: eight
    // consecutive floats per k-block, loaded as two float4 (all issued
    // before any is used; rows past the chunk read row 0 and are zeroed).
    half8 qh[NKB], ql[NKB];
    {
        const float *qr = a.q + (rvalid ? qrow : (uint64_t)a.btok0[b] * a.nh + (int)g * REP) * DK + 8 * jh;
        float4 qv[NKB][2];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            qv[kb][0] = *reinterpret_cast<const float4 *>(qr + 16 * kb);
            qv[kb][1] = *reinterpret_cast<const float4 *>(qr + 16 * kb + 4);
        }
        const float qs = rvalid ? a.qscale : 0.0f;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const float xs[8] = {qv[kb][0].x, qv[kb][0].y, qv[kb][0].z, qv[kb][0].w,
                                 qv[kb][1].x, qv[kb][1].y, qv[kb][1].z, qv[kb][1].w};
#pragma unroll
            for (int s = 0; s < 8; s++) {
                // hi and lo must both derive from the one rounded fp32 x;
                // the empty asm keeps the compiler from rounding the exact
                // product straight to fp16 for one of them (fused
                // multiply-convert), which would pair lo with another hi
                float x = xs[s] * qs;
                asm volatile("" : "+v"(x));
                const _Float16 hi = (_Float16)x;
                qh[kb][s] = hi;
                ql[kb][s] = (_Float16)(x - (float)hi);
            }
        }
    }

    // rows of this tile: keys up to the last valid row's position
    const int last_r = min(r0 + ROWS, nrows) - 1;
    const int kmax = pos + last_r / REP + 1;        // keys [0, kmax) are touched
    const int kfull = pos + r0 / REP + 1;           // keys [0, kfull) visible to every row

    float16v acc0 = {}, acc1 = {};
    float m = -FLT_MAX, lsum = 0.0f;

    const int32_t *own_pages = a.page_table + (uint64_t)seq * a.pg.pages_per_seq;
    const int32_t *pre_pages = sd.prefix >= 0 ? a.prefix_pages + (uint64_t)sd.prefix * a.pg.pages_per_seq
                                              : nullptr;
    const int P = 1 << a.pg.log2_page;

    // Chunk c of a tile: K chunks [key][KC] first, then V chunks [key][VC].
    // Page ids of a tile are fetched one iteration before its data, so no
    // data load waits on a page-table round trip.
    struct PageRef {
        int32_t page[T::CPT];
        int off[T::CPT];
    };
    auto fetch_pages = [&](int kt, PageRef &pr) {
#pragma unroll
        for (int i = 0; i < T::CPT; i++) {
            const int c = tid + i * NTHR;
            const bool isv = c >= PF_KT * T::KC;
            const int cc = isv ? c - PF_KT * T::KC : c;
            const int kl = isv ? cc / T::VC : cc / T::KC;
            const int key = kt + kl;
            pr.page[i] = -1;
            pr.off[i] = 0;
            if (c < T::NCHUNK && key < kmax) {
                if (key < n_sh) {
                    pr.page[i] = pre_pages[key >> a.pg.log2_page];
                    pr.off[i] = key & (P - 1);
                } else {
                    const int sl = key - n_sh;
                    pr.page[i] = own_pages[sl >> a.pg.log2_page];
                    pr.off[i] = sl & (P - 1);
                }
            }
        }
    };
    auto load_tile = [&](const PageRef &pr, Staged<T::CPT> &sg) {
#pragma unroll
        for (int i = 0; i < T::CPT; i++) {
            const int c = tid + i * NTHR;
            const bool isv = c >= PF_KT * T::KC;
            const int cc = isv ? c - PF_KT * T::KC : c;
            const int ch = isv ? cc % T::VC : cc % T::KC;
            sg.w[i] = u32x4{0u, 0u, 0u, 0u};
            sg.sc[i] = 0.0f;
            if (pr.page[i] >= 0) {
                const int off = pr.off[i];
                // a page is under 4 GiB: one 32 x 32 -> 64-bit multiply-add
                const uint8_t *hb = a.pool + (uint64_t)(uint32_t)pr.page[i] * (uint32_t)a.pg.page_bytes +
                                    (uint64_t)g * a.pg.head_bytes;
                const uint8_t *src = isv ? hb + (uint64_t)P * DK * ES + (uint64_t)off * DV * ES
                                         : hb + (uint64_t)off * DK * ES;
                sg.w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src) + ch);
                if (ES == 1 && ch == 0)
                    sg.sc[i] = reinterpret_cast<const float *>(hb + (uint64_t)P * (DK + DV))[(isv ? P : 0) + off];
            }
        }
    };
    auto store_tile = [&](const Staged<T::CPT> &sg, int buf) {
        _Float16 (*Ks)[T::KPAD] = Ks2[buf];
        _Float16 (*Vt)[T::VPAD] = Vt2[buf];
        float *Ksc = Ksc2[buf], *Vsc = Vsc2[buf];
#pragma unroll
        for (int i = 0; i < T::CPT; i++) {
            const int c = tid + i * NTHR;
            if (c >= T::NCHUNK)
                continue;
            const bool isv = c >= PF_KT * T::KC;
            const int cc = isv ? c - PF_KT * T::KC : c;
            const int kl = isv ? cc / T::VC : cc / T::KC;
            const int ch = isv ? cc % T::VC : cc % T::KC;
            if (!isv) {
                if constexpr (ES == 2) {
                    *reinterpret_cast<u32x4 *>(&Ks[kl][ch * 8]) = sg.w[i];
                } else {
                    half8 lo, hi;
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        lo[e] = code_at<1>(sg.w[i][e >> 2], e & 3);
                        hi[e] = code_at<1>(sg.w[i][2 + (e >> 2)], e & 3);
                    }
                    *reinterpret_cast<half8 *>(&Ks[kl][ch * 16]) = lo;
                    *reinterpret_cast<half8 *>(&Ks[kl][ch * 16 + 8]) = hi;
                    if (ch == 0)
                        Ksc[kl] = sg.sc[i];
                }
            } else {
#pragma unroll
                for (int e = 0; e < T::EPC; e++)
                    Vt[ch * T::EPC + e][kl] = code_at<ES>(sg.w[i][e / (4 / ES)], e % (4 / ES));
                if (ES == 1 && ch == 0)
                    Vsc[kl] = sg.sc[i];
            }
        }
    };

    // Register prefetch: with PD = 2, tile kt+32 waits in sg1 for its LDS
    // store while tile kt+64 loads into sg2, so each load has two tiles of
    // compute to land; the 8-wave variant keeps one tile in flight to stay
    // within the 128 registers of 4 waves per SIMD. Page ids run one tile
    // further ahead than the data.
    constexpr int PD = W >= 8 ? 1 : 2;
    Staged<T::CPT> sg1, sg2;
    PageRef pr2, pr3;
    fetch_pages(0, pr2);
    load_tile(pr2, sg1);
    store_tile(sg1, 0);
    fetch_pages(PF_KT, pr2);
    if constexpr (PD == 2) {
        load_tile(pr2, sg1);
        fetch_pages(2 * PF_KT, pr2);
    }
    __syncthreads();
    int cur = 0;
    // One key tile; `masked` is a literal at both call sites, so the
    // unmasked loop carries no diagonal-mask code at all.
    auto tile = [&](const int kt, const bool masked) __attribute__((always_inline)) {
        const bool more = kt + PF_KT < kmax;
        // No `more` guard on the loads: page ids past kmax are -1, so such a
        // tile loads nothing, and every path waits for the page ids at the
        // same point (a guarded load left a path on which the wait moved
        // behind the just-issued tile load).
        if constexpr (PD == 2) {
            load_tile(pr2, sg2);            // tile kt+64
            fetch_pages(kt + 3 * PF_KT, pr3);
        } else {
            load_tile(pr2, sg1);            // tile kt+32
            fetch_pages(kt + 2 * PF_KT, pr3);
        }
        const _Float16 (*Ks)[T::KPAD] = Ks2[cur];
        const _Float16 (*Vt)[T::VPAD] = Vt2[cur];
        const float *Ksc = Ksc2[cur], *Vsc = Vsc2[cur];

        // ---- S^T = K . Q^T (keys x rows), accumulate hi then lo
        float16v st = {};
        // Wave priority: normal while this wave issues its S MFMAs, raised
        // from the softmax through the P.V MFMAs, so a wave with softmax
        // work wins issue over waves still in their S chains (4% on a
        // 512-token chunk over 8K-32K keys; a ping-pong of half the waves one
        // phase behind, tried against it, lost 8-15%). The softmax is on
        // each tile's critical path, so its cross-half max takes a lane swap
        // (5% over an LDS permute).
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const half8 ka = *reinterpret_cast<const half8 *>(&Ks[ln][16 * kb + 8 * jh]);
            st = mfma32(ka, qh[kb], st);
            st = mfma32(ka, ql[kb], st);
        }
        __builtin_amdgcn_s_setprio(1);
        // register i holds key 8*(i/4) + 4*jh + (i%4) of the tile, row ln.
        // Only tiles crossing the diagonal mask (a work-group-uniform branch);
        // rows past the chunk compute on zero queries and are never written.
        if constexpr (ES == 1) {
#pragma unroll
            for (int i = 0; i < 16; i++)
                st[i] *= Ksc[8 * (i >> 2) + 4 * jh + (i & 3)];
        }
        if (masked) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int kl = 8 * (i >> 2) + 4 * jh + (i & 3);
                st[i] = kt + kl > qpos ? -INFINITY : st[i];
            }
        }
        // tile max over the 16 scores and the partner lane's, on 3-input
        // maxes (fmaxf would first make NaN-quieting copies of its inputs;
        // scores are never NaN)
        float mt = st[0];
#pragma unroll
        for (int i = 1; i < 15; i += 2)
            mt = max3(mt, st[i], st[i + 1]);
        mt = max3(mt, st[15], st[15]);
        {
            // the partner half's max without an LDS round trip: the swap
            // returns (own, partner) in lanes 0-31 and (partner, own) in 32-63
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = max3(mt, __uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        // Lazy max: keep the running max unless the tile exceeds it by more
        // than 2^8 (weights stay <= 256, exact range for fp16 and fp32), and
        // skip the rescale sweep when no row of the wave moved.
        const bool grow = mt > m + 8.0f;
        if (__builtin_expect(__ballot(grow) != 0, 0)) {
            const float mnew = grow ? mt : m;
            const float rs = fast_exp2(m - mnew);
            m = mnew;
            lsum *= rs;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                acc0[i] *= rs;
                acc1[i] *= rs;
            }
        }
        // P^T operand (hi, lo) for the two 16-key blocks: slots = registers
        // 8*kb2 + s. hi = p rounded toward zero to fp16, lo = the remainder.
        u32x4 phw[2], plw[2];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            float p0 = fast_exp2(st[i] - m), p1 = fast_exp2(st[i + 1] - m);
            lsum += p0 + p1;
            if constexpr (ES == 1) {
                p0 *= Vsc[8 * (i >> 2) + 4 * jh + (i & 3)];
                p1 *= Vsc[8 * (i >> 2) + 4 * jh + ((i + 1) & 3)];
            }
            const fp16x2 h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
            const uint32_t hw = __builtin_bit_cast(uint32_t, h);
            // lo = fp16(p - hi): one mixed-precision FMA per element, the fp16
            // hi half widened inside the FMA, written into its half of lw.
            uint32_t lw;
            asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(lw) : "v"(hw), "v"(p0));
            asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(lw) : "v"(hw), "v"(p1));
            phw[i >> 3][(i & 7) >> 1] = hw;
            plw[i >> 3][(i & 7) >> 1] = lw;
        }
        half8 ph[2], pl[2];
        ph[0] = __builtin_bit_cast(half8, phw[0]);
        ph[1] = __builtin_bit_cast(half8, phw[1]);
        pl[0] = __builtin_bit_cast(half8, plw[0]);
        pl[1] = __builtin_bit_cast(half8, plw[1]);
        // ---- O^T += V^T . P^T; V^T slots = keys 16*kb2 + 8*(s/4) + 4*jh + (s%4)
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++) {
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                const _Float16 *vr = &Vt[32 * dt + ln][16 * kb2 + 4 * jh];
                const half4 v0 = *reinterpret_cast<const half4 *>(vr);
                const half4 v1 = *reinterpret_cast<const half4 *>(vr + 8);
                const half8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                if (dt == 0) {
                    acc0 = mfma32(va, ph[kb2], acc0);
                    acc0 = mfma32(va, pl[kb2], acc0);
                } else {
                    acc1 = mfma32(va, ph[kb2], acc1);
                    acc1 = mfma32(va, pl[kb2], acc1);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        if (more)
            store_tile(sg1, cur ^ 1);       // tile kt+32 into the other buffer (its readers are done)
        if constexpr (PD == 2)
            sg1 = sg2;
        pr2 = pr3;
        __syncthreads();
        cur ^= 1;
    };
    // tiles [0, kfull_end) are visible to every row of the work-group
    const int kfull_end = min((kfull / PF_KT) * PF_KT, kmax);
    int kt = 0;
    for (; kt < kfull_end; kt += PF_KT)
        tile(kt, false);
    for (; kt < kmax; kt += PF_KT)
        tile(kt, true);

    // ---- emit: lane holds row ln, dims 32*dt + 8*(i/4) + 4*jh + (i%4)
    lsum += __shfl_xor(lsum, 32, 64);
    if (!rvalid)
        return;
    const float inv = 1.0f / lsum;
    float *o = a.out + qrow * DV;
    const float *gt = a.gate ? a.gate + qrow * DV : nullptr;
#pragma unroll
    for (int dt = 0; dt < 2; dt++) {
#pragma unroll
        for (int i4 = 0; i4 < 4; i4++) {
            const int d0 = 32 * dt + 8 * i4 + 4 * jh;
            float4 z;
            const float16v &acc = dt == 0 ? acc0 : acc1;
            z.x = acc[4 * i4 + 0] * inv;
            z.y = acc[4 * i4 + 1] * inv;
            z.z = acc[4 * i4 + 2] * inv;
            z.w = acc[4 * i4 + 3] * inv;
            if (gt) {
                z.x *= sigmoid_dev(gt[d0 + 0]);
                z.y *= sigmoid_dev(gt[d0 + 1]);
                z.z *= sigmoid_dev(gt[d0 + 2]);
                z.w *= sigmoid_dev(gt[d0 + 3]);
            }
            *reinterpret_cast<float4 *>(o + d0) = z;
        }
    }
}

#define NDA_PF_GEOMETRIES(X) \
    X(2, 64, 64, 1) X(2, 64, 64, 2) X(2, 64, 64, 4) X(2, 64, 64, 6) X(2, 64, 64, 8) \
    X(2, 48, 64, 1) X(2, 48, 64, 2) X(2, 48, 64, 6) \
    X(1, 64, 64, 1) X(1, 64, 64, 2) X(1, 64, 64, 4) X(1, 64, 64, 6) X(1, 64, 64, 8) \
    X(1, 48, 64, 1) X(1, 48, 64, 2) X(1, 48, 64, 6)

// Geometries whose 8-wave variant fits the 128-register budget of 4 waves per
// SIMD; the others run 4-wave work-groups.
static bool pf_w8_fits(const Geo &g) { return g.kv_f16 && g.rep == 1; }

hipError_t launch_prefill(const Geo &g, const PrefillArgs &a, int waves, hipStream_t s)
{
    if (a.n_items == 0)
        return hipSuccess;
    if (waves == 8 && !pf_w8_fits(g))
        waves = 4;
    const int es = g.kv_f16 ? 2 : 1;
    dim3 grid(a.n_items);     // n_items: a multiple of 8 (padded with empty items)
#define X(ES, DK, DV, REP)                                                                      \
    if (es == ES && g.dk == DK && g.dv == DV && g.rep == REP) {                                 \
        if (waves == 2)                                                                          \
            hipLaunchKernelGGL((prefill_kernel<ES, DK, DV, REP, 2>), grid, dim3(128), 0, s, a);  \
        else if (waves == 8)                                                                     \
            hipLaunchKernelGGL((prefill_kernel<ES, DK, DV, REP, 8>), grid, dim3(512), 0, s, a);  \
        else                                                                                     \
            hipLaunchKernelGGL((prefill_kernel<ES, DK, DV, REP, 4>), grid, dim3(256), 0, s, a);  \
        return hipGetLastError();                                                                \
    }
    NDA_PF_GEOMETRIES(X)
#undef X
    return hipErrorNotSupported;
}

} // namespace nda
