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

// Everything here is plain code the backend can see: it owes wait states
// between a VALU write and an MFMA or v_permlane32_swap read of the same
// VGPR (two on gfx950), and it cannot count them across an inline-asm
// instruction. An asm v_fma_mixhi_f16 feeding an MFMA operand got one wait
// state, so the MFMA read whatever the register held before: a stale lo half
// of P, which gave results that depended on register allocation.
//
// The tree of maxes becomes v_max3_f32 (scores are never NaN).
__device__ __forceinline__ float max3(float a, float b, float c)
{
    return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
}

// -1.0f that the optimiser cannot see through (one SGPR per kernel, so it
// costs no VGPR): with it, fma(hi, neg1, p) stays an fma over a widened fp16
// operand and is selected as one v_fma_mixlo/mixhi_f16 per value; with a
// literal -1 it is folded into a subtraction and costs a conversion, a
// subtraction and a packing.
__device__ __forceinline__ float opaque_neg1()
{
    float n = -1.0f;
    asm volatile("" : "+s"(n));
    return n;
}

// lo halves of a pair of softmax weights whose hi halves (rounded toward zero
// to fp16) are packed in hw: fp16(p - hi), rounded to nearest. p - hi is
// exact in fp32, so the one rounding is the conversion to fp16.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t split_lo2(uint32_t hw, float p0, float p1, float neg1)
{
    const half2v h = __builtin_bit_cast(half2v, hw);
    half2v l;
    l[0] = (_Float16)__builtin_fmaf((float)h[0], neg1, p0);
    l[1] = (_Float16)__builtin_fmaf((float)h[1], neg1, p1);
    return __builtin_bit_cast(uint32_t, l);
}

__device__ __forceinline__ float16v mfma32(half8 a, half8 b, float16v c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
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


// One thread's part in moving key tiles from the page pool to LDS: chunk
// c = tid + i * NTHR of a tile, K chunks [key][KC] first, then V chunks
// [key][VC]. Every load is issued, from clamped indexes: a key past kmax
// reads key kmax-1 (a stored position, so finite data that the causal mask
// and a zero weight remove) and a thread past the last chunk reads the last
// chunk, and never stores it. With no conditional loads, no loaded value is
// needed before its use a stage later, so the in-order load counter drains
// only old loads.
template <int ES, int DK, int DV, int NTHR>
struct PfIO {
    using T = PfTile<ES, DK, DV, NTHR>;
    struct PageRef {
        int32_t page[T::CPT];
        int off[T::CPT];
    };
    const uint8_t *pool;
    const int32_t *own_pages, *pre_pages;
    uint32_t page_bytes, head_bytes, log2_page, g;
    int tid, kmax, n_sh;

    __device__ __forceinline__ void fetch_pages(int kt, PageRef &pr) const
    {
        const int P = 1 << log2_page;
#pragma unroll
        for (int i = 0; i < T::CPT; i++) {
            const int c = min(tid + i * NTHR, T::NCHUNK - 1);
            const bool isv = c >= PF_KT * T::KC;
            const int cc = isv ? c - PF_KT * T::KC : c;
            const int kl = isv ? cc / T::VC : cc / T::KC;
            const int key = min(kt + kl, kmax - 1);
            const bool sh = key < n_sh;
            const int sl = sh ? key : key - n_sh;
            pr.page[i] = (sh ? pre_pages : own_pages)[sl >> log2_page];
            pr.off[i] = sl & (P - 1);
        }
    }
    __device__ __forceinline__ void load(const PageRef &pr, Staged<T::CPT> &sg) const
    {
        const int P = 1 << log2_page;
#pragma unroll
        for (int i = 0; i < T::CPT; i++) {
            const int c = min(tid + i * NTHR, T::NCHUNK - 1);
            const bool isv = c >= PF_KT * T::KC;
            const int cc = isv ? c - PF_KT * T::KC : c;
            const int ch = isv ? cc % T::VC : cc % T::KC;
            const int off = pr.off[i];
            // a page is under 4 GiB: one 32 x 32 -> 64-bit multiply-add
            const uint8_t *hb = pool + (uint64_t)(uint32_t)pr.page[i] * page_bytes + (uint64_t)g * head_bytes;
            const uint8_t *src = isv ? hb + (uint64_t)P * DK * ES + (uint64_t)off * DV * ES
                                     : hb + (uint64_t)off * DK * ES;
            sg.w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src) + ch);
            if constexpr (ES == 1)
                sg.sc[i] = reinterpret_cast<const float *>(hb + (uint64_t)P * (DK + DV))[(isv ? P : 0) + off];
            else
                sg.sc[i] = 0.0f;
        }
    }
    __device__ __forceinline__ void store(const Staged<T::CPT> &sg, _Float16 (*Ks)[T::KPAD],
                                          _Float16 (*Vt)[T::VPAD], float *Ksc, float *Vsc) const
    {
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
    }
};

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
    const float neg1 = opaque_neg1();

    PfIO<ES, DK, DV, NTHR> io;
    io.pool = a.pool;
    io.own_pages = a.page_table + (uint64_t)seq * a.pg.pages_per_seq;
    io.pre_pages = sd.prefix >= 0 ? a.prefix_pages + (uint64_t)sd.prefix * a.pg.pages_per_seq : nullptr;
    io.page_bytes = a.pg.page_bytes;
    io.head_bytes = a.pg.head_bytes;
    io.log2_page = a.pg.log2_page;
    io.g = g;
    io.tid = tid;
    io.kmax = kmax;
    io.n_sh = n_sh;
    const int ntile = (kmax + PF_KT - 1) / PF_KT;
    const int jfull = min(kfull / PF_KT, ntile);    // tiles [0, jfull) visible to every row

    // Register prefetch: with PD = 2, tile j+1 waits in registers for its
    // LDS store while tile j+2 loads, so each load has two tiles of compute
    // to land; the 8-wave variant keeps one tile in flight to stay within the
    // 128 registers of 4 waves per SIMD. Tiles in flight and their page ids
    // sit in rings indexed by tile parity (a register copy would wait on the
    // newest load), and a tile's page ids are fetched before the data load
    // issued beside them, so waiting for ids fetched a tile earlier never
    // waits for the data load that followed them.
    constexpr int PD = W >= 8 ? 1 : 2;
    typename PfIO<ES, DK, DV, NTHR>::PageRef prn[2];
    Staged<T::CPT> sg[PD];
    io.fetch_pages(0, prn[0]);
    io.fetch_pages(PF_KT, prn[1]);
    io.load(prn[0], sg[0]);                     // tile 0
    io.store(sg[0], Ks2[0], Vt2[0], Ksc2[0], Vsc2[0]);
    io.fetch_pages(2 * PF_KT, prn[0]);
    io.load(prn[1], sg[1 % PD]);                // tile 1
    if constexpr (PD == 2) {
        io.fetch_pages(3 * PF_KT, prn[1]);
        io.load(prn[0], sg[0]);                 // tile 2
    }
    __syncthreads();

    // One key tile j (parity PJ = j & 1); the LDS buffer of tile j is PJ.
    // `masked` is a compile-time flag: the loop over tiles below the
    // diagonal carries no mask code (whose registers would spill the 8-wave
    // variant). With fp16 K/V the S MFMAs of every tile after the first
    // start from -m, so they return s - m and the exps need no subtraction
    // (the first tile, with no running max yet, starts from zero).
    auto tile = [&](const int j, auto pj, auto masked, auto first) __attribute__((always_inline)) {
        constexpr int PJ = decltype(pj)::value, Q1 = PJ ^ 1;
        constexpr bool REL = ES == 2 && !decltype(first)::value;   // scores relative to m
        const int kt = j * PF_KT;
        // ids of tile j+PD+1 into the slot of tile j+PD-1's (spent), then the
        // data of tile j+PD; past kmax the loads read the last key (finite
        // data, masked)
        io.fetch_pages((j + PD + 1) * PF_KT, prn[(PJ + PD + 1) & 1]);
        io.load(prn[(PJ + PD) & 1], sg[(PJ + PD) % PD]);
        const _Float16 (*Ks)[T::KPAD] = Ks2[PJ];
        const _Float16 (*Vt)[T::VPAD] = Vt2[PJ];
        const float *Ksc = Ksc2[PJ], *Vsc = Vsc2[PJ];

        // ---- S^T = K . Q^T (keys x rows), accumulate hi then lo
        float16v st;
#pragma unroll
        for (int i = 0; i < 16; i++)
            st[i] = REL ? -m : 0.0f;
        // Wave priority: normal while this wave issues its S MFMAs, raised
        // from the softmax through the P.V MFMAs, so a wave with softmax
        // work wins issue over waves still in their S chains (4% on a
        // 512-token chunk over 8K-32K keys). A ping-pong of two waves per
        // SIMD, one in its MFMAs while the other runs its softmax, lost 3%
        // against it: with one work-group per CU, latency the four resident
        // waves hide here stays exposed. The softmax is on each tile's
        // critical path, so its cross-half max takes a lane swap (5% over an
        // LDS permute) and its max and sum are trees.
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
        if constexpr (decltype(masked)::value) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int kl = 8 * (i >> 2) + 4 * jh + (i & 3);
                st[i] = kt + kl > qpos ? -INFINITY : st[i];
            }
        }
        // tile max over the 16 scores (a tree of 3-input maxes: fmaxf would
        // first make NaN-quieting copies of its inputs; scores are never NaN)
        // and the partner lane's, without an LDS round trip: the swap
        // returns (own, partner) in lanes 0-31 and (partner, own) in 32-63
        const float x0 = max3(st[0], st[1], st[2]), x1 = max3(st[3], st[4], st[5]);
        const float x2 = max3(st[6], st[7], st[8]), x3 = max3(st[9], st[10], st[11]);
        const float x4 = max3(st[12], st[13], st[14]);
        const float y0 = max3(x0, x1, x2), y1 = max3(x3, x4, st[15]);
        float mt = max3(y0, y1, y1);
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = max3(mt, __uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        // Lazy max: keep the running max unless the tile exceeds it by more
        // than 2^8 (weights stay <= 256, exact range for fp16 and fp32), and
        // skip the rescale sweep when no row of the wave moved.
        const bool grow = REL ? mt > 8.0f : mt > m + 8.0f;
        if (__builtin_expect(__ballot(grow) != 0, 0)) {
            if constexpr (REL) {
                const float d = grow ? mt : 0.0f;     // the running max moves by d
                const float rs = fast_exp2(-d);
                m += d;
                lsum *= rs;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    acc0[i] *= rs;
                    acc1[i] *= rs;
                    st[i] -= d;
                }
            } else {
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
        }
        // P^T operand (hi, lo) and O^T += V^T . P^T, one 16-key block at a
        // time (keys 16*kb2 + 8*(s/4) + 4*jh + (s%4) in slot s): a block's
        // weights are made just before its MFMAs, which keeps their live
        // ranges short. hi = p rounded toward zero to fp16, lo = the remainder.
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++) {
            u32x4 phw, plw;
#pragma unroll
            for (int i = 8 * kb2; i < 8 * kb2 + 8; i += 2) {
                float p0 = fast_exp2(REL ? st[i] : st[i] - m), p1 = fast_exp2(REL ? st[i + 1] : st[i + 1] - m);
                lsum += p0 + p1;
                if constexpr (ES == 1) {
                    p0 *= Vsc[8 * (i >> 2) + 4 * jh + (i & 3)];
                    p1 *= Vsc[8 * (i >> 2) + 4 * jh + ((i + 1) & 3)];
                }
                const fp16x2 h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
                const uint32_t hw = __builtin_bit_cast(uint32_t, h);
                phw[(i & 7) >> 1] = hw;
                plw[(i & 7) >> 1] = split_lo2(hw, p0, p1, neg1);
            }
            const half8 ph = __builtin_bit_cast(half8, phw), pl = __builtin_bit_cast(half8, plw);
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                const _Float16 *vr = &Vt[32 * dt + ln][16 * kb2 + 4 * jh];
                const half4 v0 = *reinterpret_cast<const half4 *>(vr);
                const half4 v1 = *reinterpret_cast<const half4 *>(vr + 8);
                const half8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                if (dt == 0) {
                    acc0 = mfma32(va, ph, acc0);
                    acc0 = mfma32(va, pl, acc0);
                } else {
                    acc1 = mfma32(va, ph, acc1);
                    acc1 = mfma32(va, pl, acc1);
                }
            }
            if (kb2 == 0)
                __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
        if (j + 1 < ntile)   // tile j+1 into the other buffer (its readers are done)
            io.store(sg[(PJ + 1) % PD], Ks2[Q1], Vt2[Q1], Ksc2[Q1], Vsc2[Q1]);
        __syncthreads();
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using Full = std::false_type;
    using Diag = std::true_type;
    using First = std::true_type;
    using Next = std::false_type;
    // Pairs of tiles keep each parity static, the first pair holding the
    // first tile (whose running max starts from its own scores). The
    // unmasked loop stops at an even tile, so the masked loop starts on
    // parity 0 as well (a visible tile taken into it masks nothing). (A
    // variant that peeled tile 0 and paired (odd, even) tiles after it gave
    // wrong int8 results with two tiles in flight; this order is the tested
    // one.)
    const int jeven = jfull & ~1;
    int j;
    if (jeven >= 2) {
        tile(0, P0{}, Full{}, First{});
        tile(1, P1{}, Full{}, Next{});
        j = 2;
    } else if (ntile >= 2) {
        tile(0, P0{}, Diag{}, First{});
        tile(1, P1{}, Diag{}, Next{});
        j = 2;
    } else {
        tile(0, P0{}, Diag{}, First{});
        j = 1;
    }
    for (; j < jeven; j += 2) {
        tile(j, P0{}, Full{}, Next{});
        tile(j + 1, P1{}, Full{}, Next{});
    }
    for (; j + 1 < ntile; j += 2) {
        tile(j, P0{}, Diag{}, Next{});
        tile(j + 1, P1{}, Diag{}, Next{});
    }
    if (j < ntile)
        tile(j, P0{}, Diag{}, Next{});

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

// ------------------------------------------------------------ GQA decode
//
// Decode of a GQA group (rep >= 4) on MFMA: one wave per (row, kv-head), the
// group's rep query heads as the wave's rows (32 row slots, rep of them
// valid), every visible slot as its keys, in slot order (sinks, shared
// prefix and ring alike; softmax does not depend on the order, and the
// visible set is the engine's, engine/src/nd_model.c:2451-2483). The tile
// arithmetic is the prefill kernel's (S^T = K.Q^T and O^T += V^T.P^T with
// fp16 hi + lo operands, the lazy running max); only keys past the last
// visible slot are masked. The per-lane dot products, lane reductions and
// fp32 conversions that bound the VALU decode kernel at this shape move to
// the matrix cores.
//
// Staging: lane (ln, jh) moves half jh of key ln of a 32-key tile (K codes
// [DK/2 jh, +DK/2), V codes [32 jh, +32) and the key's K (jh 0) or V (jh 1)
// scale), so each lane needs one page id a tile, fetched a tile ahead. The
// loads are unconditional (a key past the last visible slot reads the last
// one: finite data, masked). int8 codes become fp16 exactly with one byte
// permute and one packed fp16 subtract per two codes: 0x64 over the byte
// (code ^ 0x80) is the fp16 1024 + code + 128. One wave owns its LDS tile,
// whose accesses complete in order, so one buffer serves.
template <int SEL>
__device__ __forceinline__ half2v codes2(uint32_t xs)   // xs = codes ^ 0x80808080
{
    const uint32_t u = __builtin_amdgcn_perm(0x64646464u, xs, (uint32_t)SEL);
    return __builtin_bit_cast(half2v, u) - half2v{(_Float16)1152.0f, (_Float16)1152.0f};
}

typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4v mfma16k32(half8 a, half8 b, float4v c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16 x 16 tiles: lane l = 16 g + r holds MFMA row / column r and the k (or
// output row) slots of lane group g. A wave's 16 row slots hold the group's
// rep heads; a 32-key tile is two 16-key blocks of S^T = K.Q^T (lane: row r,
// keys 16 b + 4 g + i), whose eight scores per lane are, in that order, the
// P^T operand of O^T += V^T.P^T over the 32 keys (lane group g's k slots),
// so V^T is read in the same key order. A row's softmax state spans the four
// lane groups (a max and a sum across them).
template <int DK, int DV, int REP>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4)))
void decode_mfma_kernel(PrefillArgs a)
{
    static_assert(DK % 16 == 0 && DV == 64 && REP <= 16, "decode tiles: dk multiple of 16, dv 64, rep <= 16");
    constexpr int NS = DK / 32;                 // 32-dim steps of S (16x16x32)
    // A last 16-dim step (qk 48) runs on the same 16x16x32 instruction, its
    // upper four k slots zero in both operands. Every accumulation chain
    // thus keeps one opcode: an MFMA reading as its accumulator the result
    // of the MFMA issued just before it, of another opcode (16x16x16 after
    // 16x16x32), gave wrong results on gfx950 although the compiler puts no
    // wait state between them, as it does for the same opcode.
    constexpr bool TAIL = DK % 32 == 16;
    constexpr int KPAD = DK + 8, VPAD = PF_KT + 4;
    constexpr int KH = DK / 2, VH = DV / 2;     // codes a lane moves per key
    static_assert(KH % 8 == 0 && VH % 16 == 0, "lane halves are whole 8- and 16-byte loads");
    __shared__ __attribute__((aligned(16))) _Float16 Ks[PF_KT][KPAD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[DV][VPAD];
    __shared__ __attribute__((aligned(16))) float Sc[2][PF_KT];   // K, V scales of the tile's keys

    const int lane = threadIdx.x;
    const int jh = lane >> 5, ln = lane & 31;   // staging: key ln, half jh
    const int g = lane >> 4, r = lane & 15;     // MFMA: lane group, row / column
    const uint32_t nkv = a.pg.nkv;
    const uint32_t b = blockIdx.x / nkv, kvh = blockIdx.x % nkv;
    const uint32_t seq = a.row_seq ? a.row_seq[b] : b;
    const SeqDev sd = a.seqs[seq];
    const Visible vis = visible(sd, sd.pos, (int)a.pg.window);
    const int n_sh = vis.n_sh, total = vis.n_sh + vis.n_own;

    // Q^T operand, hi and lo: row r, dims 32 s + 8 g + [0, 8) and the tail
    // 32 NS + 4 g + [0, 4) (then four zero slots); hi and lo from one rounded
    // fp32 value
    const bool rvalid = r < REP;
    const uint64_t qrow = (uint64_t)b * a.nh + kvh * REP + (rvalid ? r : 0);
    half8 qh[NS > 0 ? NS : 1], ql[NS > 0 ? NS : 1];
    half8 qht = {}, qlt = {};
    {
        const float *qr = a.q + qrow * DK;
        const float qs = rvalid ? a.qscale : 0.0f;
        auto split = [&](float v, _Float16 &hi, _Float16 &lo) __attribute__((always_inline)) {
            float x = v * qs;
            asm volatile("" : "+v"(x));
            hi = (_Float16)x;
            lo = (_Float16)(x - (float)hi);
        };
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const float4 v0 = *reinterpret_cast<const float4 *>(qr + 32 * st + 8 * g);
            const float4 v1 = *reinterpret_cast<const float4 *>(qr + 32 * st + 8 * g + 4);
            const float xs[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                _Float16 hi, lo;
                split(xs[i], hi, lo);
                qh[st][i] = hi;
                ql[st][i] = lo;
            }
        }
        if constexpr (TAIL) {
            const float4 v = *reinterpret_cast<const float4 *>(qr + 32 * NS + 4 * g);
            const float xs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                _Float16 hi, lo;
                split(xs[i], hi, lo);
                qht[i] = hi;
                qlt[i] = lo;
            }
        }
    }

    const int P = 1 << a.pg.log2_page;
    const int32_t *own = a.page_table + (uint64_t)seq * a.pg.pages_per_seq;
    const int32_t *pre = sd.prefix >= 0 ? a.prefix_pages + (uint64_t)sd.prefix * a.pg.pages_per_seq : own;
    // page id (loaded) and in-page offset of this lane's key of tile j
    auto fetch = [&](int j, int32_t &pid, int &off) __attribute__((always_inline)) {
        const int key = min(j * PF_KT + ln, total - 1);
        const bool sh = key < n_sh;
        const int sl = sh ? key : key - n_sh;
        pid = (sh ? pre : own)[sl >> a.pg.log2_page];
        off = sl & (P - 1);
    };
    struct Stage {
        uint32_t k[KH / 4], v[VH / 4];
        float sc;
    };
    auto load = [&](int32_t pid, int off, Stage &sg) __attribute__((always_inline)) {
        // a page is under 4 GiB: one 32 x 32 -> 64-bit multiply-add
        const uint8_t *hb = a.pool + (uint64_t)(uint32_t)pid * (uint32_t)a.pg.page_bytes + (uint64_t)kvh * a.pg.head_bytes;
        const uint8_t *kp = hb + off * DK + KH * jh;
        const uint8_t *vp = hb + P * DK + off * DV + VH * jh;
#pragma unroll
        for (int i = 0; i < KH / 8; i++) {
            const u32x2 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(kp) + i);
            sg.k[2 * i] = x.x;
            sg.k[2 * i + 1] = x.y;
        }
#pragma unroll
        for (int i = 0; i < VH / 16; i++) {
            const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vp) + i);
            sg.v[4 * i] = x.x;
            sg.v[4 * i + 1] = x.y;
            sg.v[4 * i + 2] = x.z;
            sg.v[4 * i + 3] = x.w;
        }
        sg.sc = reinterpret_cast<const float *>(hb + P * (DK + DV))[jh * P + off];
    };
    auto store = [&](const Stage &sg) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KH / 8; i++) {
            const uint32_t x0 = sg.k[2 * i] ^ 0x80808080u, x1 = sg.k[2 * i + 1] ^ 0x80808080u;
            const half2v c0 = codes2<0x04010400>(x0), c1 = codes2<0x04030402>(x0);
            const half2v c2 = codes2<0x04010400>(x1), c3 = codes2<0x04030402>(x1);
            *reinterpret_cast<half8 *>(&Ks[ln][KH * jh + 8 * i]) =
                half8{c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
        }
#pragma unroll
        for (int i = 0; i < VH / 4; i++) {
            const uint32_t x = sg.v[i] ^ 0x80808080u;
            const half2v c0 = codes2<0x04010400>(x), c1 = codes2<0x04030402>(x);
            Vt[VH * jh + 4 * i + 0][ln] = c0[0];
            Vt[VH * jh + 4 * i + 1][ln] = c0[1];
            Vt[VH * jh + 4 * i + 2][ln] = c1[0];
            Vt[VH * jh + 4 * i + 3][ln] = c1[1];
        }
        Sc[jh][ln] = sg.sc;
    };

    float4v acc[4] = {};                        // O^T: dims 16 d + 4 g + i, row r
    float m = -FLT_MAX, lsum = 0.0f;
    const float neg1 = opaque_neg1();
    const int qlast = total - 1;                // keys past it are masked
    const int ntile = (total + PF_KT - 1) / PF_KT;
    const int jfull = total / PF_KT;            // tiles [0, jfull) are all visible

    int32_t pid[2];
    int poff[2];
    Stage sg;
    fetch(0, pid[0], poff[0]);
    fetch(1, pid[1], poff[1]);
    load(pid[0], poff[0], sg);
    store(sg);

    // tile j (parity PJ): ids of tile j+2 into tile j's slot, data of tile
    // j+1, the tile's arithmetic, then tile j+1 into LDS (two tiles in
    // flight measured the same: the wave's chain through a tile, not the
    // load latency, is what the resident waves hide)
    auto tile = [&](const int j, auto pj, auto masked) __attribute__((always_inline)) {
        constexpr int PJ = decltype(pj)::value, Q1 = PJ ^ 1;
        const int kt = j * PF_KT;
        fetch(j + 2, pid[PJ], poff[PJ]);
        load(pid[Q1], poff[Q1], sg);

        float4v st[2];
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const _Float16 *kr = &Ks[16 * kb + r][0];
            st[kb] = float4v{};
#pragma unroll
            for (int s2 = 0; s2 < NS; s2++) {
                const half8 ka = *reinterpret_cast<const half8 *>(kr + 32 * s2 + 8 * g);
                st[kb] = mfma16k32(ka, qh[s2], st[kb]);
                st[kb] = mfma16k32(ka, ql[s2], st[kb]);
            }
            if constexpr (TAIL) {
                const half4 k4 = *reinterpret_cast<const half4 *>(kr + 32 * NS + 4 * g);
                const half8 ka = {k4[0], k4[1], k4[2], k4[3], 0, 0, 0, 0};
                st[kb] = mfma16k32(ka, qht, st[kb]);
                st[kb] = mfma16k32(ka, qlt, st[kb]);
            }
        }
        __builtin_amdgcn_s_setprio(1);
        // scores of keys 16 kb + 4 g + i: k scales, then the mask
        {
            const float4 k0 = *reinterpret_cast<const float4 *>(&Sc[0][4 * g]);
            const float4 k1 = *reinterpret_cast<const float4 *>(&Sc[0][16 + 4 * g]);
            st[0] *= float4v{k0.x, k0.y, k0.z, k0.w};
            st[1] *= float4v{k1.x, k1.y, k1.z, k1.w};
        }
        if constexpr (decltype(masked)::value) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    st[kb][i] = kt + 16 * kb + 4 * g + i > qlast ? -INFINITY : st[kb][i];
        }
        // the row's tile max over its 32 keys: 8 in this lane, then across
        // the four lane groups (lanes r + 16 g)
        const float y0 = max3(st[0][0], st[0][1], st[0][2]), y1 = max3(st[0][3], st[1][0], st[1][1]);
        float mt = max3(y0, y1, max3(st[1][2], st[1][3], st[1][3]));
        mt = max3(mt, __shfl_xor(mt, 16, 64), mt);
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = max3(mt, __uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const bool grow = mt > m + 8.0f;
        if (__builtin_expect(__ballot(grow) != 0, 0)) {
            const float mnew = grow ? mt : m;
            const float rs = fast_exp2(m - mnew);
            m = mnew;
            lsum *= rs;
#pragma unroll
            for (int d = 0; d < 4; d++)
                acc[d] *= rs;
        }
        float p[8];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                p[4 * kb + i] = fast_exp2(st[kb][i] - m);
        lsum += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
        {
            const float4 v0 = *reinterpret_cast<const float4 *>(&Sc[1][4 * g]);
            const float4 v1 = *reinterpret_cast<const float4 *>(&Sc[1][16 + 4 * g]);
            p[0] *= v0.x; p[1] *= v0.y; p[2] *= v0.z; p[3] *= v0.w;
            p[4] *= v1.x; p[5] *= v1.y; p[6] *= v1.z; p[7] *= v1.w;
        }
        // P^T operand (hi, lo): slots = the eight keys in lane order; hi = p
        // rounded toward zero to fp16, lo = the remainder
        u32x4 phw, plw;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const fp16x2 hh = __builtin_amdgcn_cvt_pkrtz(p[i], p[i + 1]);
            const uint32_t hw = __builtin_bit_cast(uint32_t, hh);
            phw[i >> 1] = hw;
            plw[i >> 1] = split_lo2(hw, p[i], p[i + 1], neg1);
        }
        const half8 ph = __builtin_bit_cast(half8, phw), pl = __builtin_bit_cast(half8, plw);
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const _Float16 *vr = &Vt[16 * d + r][4 * g];
            const half4 v0 = *reinterpret_cast<const half4 *>(vr);
            const half4 v1 = *reinterpret_cast<const half4 *>(vr + 16);
            const half8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            acc[d] = mfma16k32(va, ph, acc[d]);
            acc[d] = mfma16k32(va, pl, acc[d]);
        }
        __builtin_amdgcn_s_setprio(0);
        // Tile j+1 into LDS after this tile's last LDS reads. Other lanes of
        // the wave read what this lane stores, and the wave's LDS accesses
        // complete in issue order; the wave barriers (scheduling barriers,
        // no instruction) keep the compiler from moving LDS accesses of one
        // tile across the store of the next.
        if (j + 1 < ntile) {
            __builtin_amdgcn_wave_barrier();
            store(sg);
            __builtin_amdgcn_wave_barrier();
        }
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    const int jeven = jfull & ~1;
    int j = 0;
    for (; j < jeven; j += 2) {
        tile(j, P0{}, std::false_type{});
        tile(j + 1, P1{}, std::false_type{});
    }
    for (; j + 1 < ntile; j += 2) {
        tile(j, P0{}, std::true_type{});
        tile(j + 1, P1{}, std::true_type{});
    }
    if (j < ntile)
        tile(j, P0{}, std::true_type{});

    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    if (!rvalid)
        return;
    const float inv = 1.0f / lsum;
    float *o = a.out + qrow * DV;
    const float *gt = a.gate ? a.gate + qrow * DV : nullptr;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int d0 = 16 * d + 4 * g;
        float4 z;
        z.x = acc[d][0] * inv;
        z.y = acc[d][1] * inv;
        z.z = acc[d][2] * inv;
        z.w = acc[d][3] * inv;
        if (gt) {
            z.x *= sigmoid_dev(gt[d0 + 0]);
            z.y *= sigmoid_dev(gt[d0 + 1]);
            z.z *= sigmoid_dev(gt[d0 + 2]);
            z.w *= sigmoid_dev(gt[d0 + 3]);
        }
        *reinterpret_cast<float4 *>(o + d0) = z;
    }
}

// GQA decode geometries of the MFMA kernel (int8 K/V, 4+ heads per kv-head)
#define NDA_DEC_GEOMETRIES(X) X(48, 64, 6) X(64, 64, 4) X(64, 64, 6) X(64, 64, 8)

bool decode_mfma_supported(const Geo &g)
{
#define X(DK, DV, REP) if (!g.kv_f16 && g.dk == DK && g.dv == DV && g.rep == REP) return true;
    NDA_DEC_GEOMETRIES(X)
#undef X
    return false;
}

hipError_t launch_decode_mfma(const Geo &g, const PrefillArgs &a, hipStream_t s)
{
    if (a.n_items == 0)
        return hipSuccess;
#define X(DK, DV, REP)                                                                            \
    if (!g.kv_f16 && g.dk == DK && g.dv == DV && g.rep == REP) {                                  \
        hipLaunchKernelGGL((decode_mfma_kernel<DK, DV, REP>), dim3(a.n_items), dim3(64), 0, s, a); \
        return hipGetLastError();                                                                 \
    }
    NDA_DEC_GEOMETRIES(X)
#undef X
    return hipErrorNotSupported;
}

#define NDA_PF_GEOMETRIES(X) \
    X(2, 64, 64, 1) X(2, 64, 64, 2) X(2, 64, 64, 4) X(2, 64, 64, 6) X(2, 64, 64, 8) \
    X(2, 48, 64, 1) X(2, 48, 64, 2) X(2, 48, 64, 6) \
    X(1, 64, 64, 1) X(1, 64, 64, 2) X(1, 64, 64, 4) X(1, 64, 64, 6) X(1, 64, 64, 8) \
    X(1, 48, 64, 1) X(1, 48, 64, 2) X(1, 48, 64, 6)

bool prefill_mfma_supported(const Geo &g)
{
#define X(ES, DK, DV, REP) if ((g.kv_f16 ? 2 : 1) == ES && g.dk == DK && g.dv == DV && g.rep == REP) return true;
    NDA_PF_GEOMETRIES(X)
#undef X
    return false;
}

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
