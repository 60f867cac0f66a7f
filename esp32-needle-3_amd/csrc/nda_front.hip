// nda_front.hip - the attention front on gfx950: what attention() does to
// the raw q/k/v projections before the KV store (engine/src/nd_model.c:
// 2413-2424):
//
//   tap_projection x3   causal depthwise convolution of every column over the
//                       last `taps` raw projections (:2361-2379, tap_rows
//                       :1748-1802): hist[pos % taps] = raw, then
//                       y[i] = sum_{j < min(taps, pos+1)} w[j][i] * x_{pos-j}[i]
//   zcrms_heads x2      per-head RMS norm of q and k with a (1 + s) scale
//                       shared by all heads, fused with GPT-NeoX half-split
//                       RoPE at the row's position (:324-360)
//
// One work-group per (row, kv-head group): a row is one token of one
// sequence, a group the rep query heads sharing one kv-head plus that k and v
// head, so every normalised head lies inside one work-group (two rows per
// work-group, front_pair_kernel, for large launches of several tokens per
// sequence). Each thread owns
// four consecutive columns and issues all its loads (the raw row, the older
// raw rows of the taps, the tap weights) before using any, so a wave keeps
// its whole working set in flight. The per-head sum of squares is a
// sequential walk by one thread per head (the reference's order); the emit is
// one (head, rotary pair) per thread. Store mode then writes the k/v rows
// into the KV pages exactly as the append kernel does (int8 with the engine's
// Markstein store, or fp16), so the decode launch that follows reads them
// from the cache.
//
// Every multiply and add rounds on its own (no contraction) and divide / sqrt
// are correctly rounded, so the results are bit-identical to the engine's
// host build, and so are the int8 codes computed from them.
#include "nda_device.h"

#include <algorithm>

namespace nda {

template <int DK, int DV, int REP>
struct FrontShape {
    static constexpr int NC = REP * DK + DK + DV;   // columns of one kv group
    static constexpr int NG = NC / 4;               // four-column groups, one per thread
    static constexpr int W = (NG + 63) / 64;        // waves per work-group
    static constexpr int NH = REP + 1;              // normalised heads: REP q + 1 k
    static constexpr int STRIDE = DK + 4;           // LDS row: 16-byte aligned, banks spread
    static constexpr int HALF = DK / 2;
    static constexpr int TREG = 4;                  // taps held in registers; more are streamed
    static_assert(DK % 4 == 0 && DV % 4 == 0, "four-column groups");
    static_assert(W <= 4, "one group per thread");
};

typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

__device__ __forceinline__ void acc4(float4 &a, const float4 &w, const float4 &x)
{
#pragma clang fp contract(off)
    a.x = a.x + w.x * x.x;
    a.y = a.y + w.y * x.y;
    a.z = a.z + w.z * x.z;
    a.w = a.w + w.w * x.w;
}

template <int ES, int DK, int DV, int REP>
__global__ __launch_bounds__((64 * FrontShape<DK, DV, REP>::W)) void front_kernel(FrontArgs a)
{
#pragma clang fp contract(off)
    using S = FrontShape<DK, DV, REP>;
    __shared__ __align__(16) float ylds[S::NH * S::STRIDE];   // conv outputs of the q/k heads
    __shared__ __align__(16) float sqlds[S::NH * S::STRIDE];  // their squares
    __shared__ __align__(16) float vlds[DV];
    __shared__ float invlds[S::NH];

    const uint32_t nkv = a.nkv;
    const uint32_t row = blockIdx.x / nkv, g = blockIdx.x % nkv;
    const int tid = threadIdx.x;
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const uint32_t t = a.row_t ? a.row_t[row] : 0u;
    const SeqDev sd = a.seqs[seq];
    const uint32_t pos = (uint32_t)sd.pos + t;
    const uint32_t taps = a.taps;
    const uint32_t nt = min(taps, pos + 1u);
    const uint32_t dq = nkv * REP * DK, dk = nkv * DK, dv = nkv * DV, dcol = dq + dk + dv;
    float *hist = a.hist + ((uint64_t)seq * a.n_layers + a.layer) * taps * dcol;
    const bool store = a.k_out == nullptr;

    // What steps 3 and 4 read (this thread's rotary pairs and norm scales,
    // the page of the stored slot) is requested now, beside the tap loads,
    // so the wave waits on one round of loads rather than three.
    constexpr int NE = (S::NH * S::HALF + 64 * S::W - 1) / (64 * S::W);   // emit elements per thread
    const float2 *rope = a.rope + (uint64_t)pos * S::HALF;
    float2 cs_e[NE];
    float s1_e[NE], s2_e[NE];
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = tid + n * 64 * S::W;
        const int h = e / S::HALF, i = e % S::HALF;
        if (e < S::NH * S::HALF) {
            const float *sn = a.norm + (h < REP ? 0 : DK);
            cs_e[n] = rope[i];
            s1_e[n] = sn[i];
            s2_e[n] = sn[i + S::HALF];
        }
    }
    int slot = 0;
    int32_t page = -1;
    if (store) {
        slot = own_slot(sd, (int)pos, (int)a.pg.window);
        page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (slot >> a.pg.log2_page)];
    }

    // 1. tap convolution of this thread's four columns
    const bool active = tid < S::NG;
    const int lc = tid * 4;                      // column within the group
    const float *src;
    uint32_t ld, cc, gc;                         // source row length, column in it, column in dcol
    if (lc < REP * DK) {
        src = a.q; ld = dq; cc = g * REP * DK + lc; gc = cc;
    } else if (lc < REP * DK + DK) {
        src = a.k; ld = dk; cc = g * DK + (lc - REP * DK); gc = dq + cc;
    } else {
        src = a.v; ld = dv; cc = g * DV + (lc - REP * DK - DK); gc = dq + dk + cc;
    }
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 raw = acc;
    if (active) {
        float4 x[S::TREG], w[S::TREG];
        raw = ld4(src + (uint64_t)row * ld + cc);
#pragma unroll
        for (int j = 0; j < S::TREG; j++) {
            if ((uint32_t)j < nt) {
                w[j] = ld4(a.w + (uint64_t)j * dcol + gc);
                if (j == 0)
                    x[j] = raw;
                else if ((uint32_t)j <= t)
                    x[j] = ld4(src + (uint64_t)(row - j) * ld + cc);
                else
                    x[j] = ld4(hist + (uint64_t)((pos - j) % taps) * dcol + gc);
            }
        }
#pragma unroll
        for (int j = 0; j < S::TREG; j++)
            if ((uint32_t)j < nt)
                acc4(acc, w[j], x[j]);
        for (uint32_t j = S::TREG; j < nt; j++) {
            const float4 wj = ld4(a.w + (uint64_t)j * dcol + gc);
            const float4 xj = j <= t ? ld4(src + (uint64_t)(row - j) * ld + cc)
                                     : ld4(hist + (uint64_t)((pos - j) % taps) * dcol + gc);
            acc4(acc, wj, xj);
        }
        // the raw row into the tap history, read again only at the next
        // step's front: streamed past L2 (2-6% off the 4096-row front)
        if (a.hist_write)
            __builtin_nontemporal_store(float4v{raw.x, raw.y, raw.z, raw.w},
                                        reinterpret_cast<float4v *>(hist + (uint64_t)(pos % taps) * dcol + gc));
        if (lc < (REP + 1) * DK) {
            const int o = (lc / DK) * S::STRIDE + lc % DK;
            *reinterpret_cast<float4 *>(ylds + o) = acc;
            *reinterpret_cast<float4 *>(sqlds + o) =
                make_float4(acc.x * acc.x, acc.y * acc.y, acc.z * acc.z, acc.w * acc.w);
        } else if (store) {
            *reinterpret_cast<float4 *>(vlds + (lc - (REP + 1) * DK)) = acc;
        } else {
            *reinterpret_cast<float4 *>(a.v_out + (uint64_t)row * dv + cc) = acc;
        }
    }
    __syncthreads();

    // 2. per-head sum of squares in index order, inverse RMS
    if (tid < S::NH) {
        const float *r = sqlds + tid * S::STRIDE;
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < DK; i++)
            ss = ss + r[i];
        invlds[tid] = 1.0f / __builtin_sqrtf(ss / (float)DK + 1e-6f);
    }
    __syncthreads();

    // 3. (1 + s) * x * inv, rotated by the position's (cos, sin)
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = tid + n * 64 * S::W;
        if (e >= S::NH * S::HALF)
            break;
        const int h = e / S::HALF, i = e % S::HALF;
        const bool is_q = h < REP;
        float *r = ylds + h * S::STRIDE;
        const float iv = invlds[h];
        const float x1 = (1.0f + s1_e[n]) * r[i] * iv;
        const float x2 = (1.0f + s2_e[n]) * r[i + S::HALF] * iv;
        const float2 cs = cs_e[n];
        const float o1 = x1 * cs.x - x2 * cs.y;
        const float o2 = x2 * cs.x + x1 * cs.y;
        if (is_q) {
            float *qo = a.q_out + (uint64_t)row * dq + (g * REP + h) * DK;
            qo[i] = o1;
            qo[i + S::HALF] = o2;
        } else if (store) {
            r[i] = o1;
            r[i + S::HALF] = o2;
        } else {
            float *ko = a.k_out + (uint64_t)row * dk + g * DK;
            ko[i] = o1;
            ko[i + S::HALF] = o2;
        }
    }
    if (!store)
        return;
    __syncthreads();

    // 4. store this position's k/v rows of kv-head g (wave 0, lane = element)
    if (tid >= 64)
        return;
    const int P = 1 << a.pg.log2_page;
    if (page < 0)
        return;   // the host backs every stored slot; never taken
    uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
    const float kx = tid < DK ? ylds[REP * S::STRIDE + tid] : 0.0f;
    const float vx = tid < DV ? vlds[tid] : 0.0f;
    store_row<ES>(hb, slot & (P - 1), P, kx, vx, tid, DK, DV);
}

// front_kernel over two rows per work-group, for launches of several tokens
// per sequence (the rows are then consecutive tokens, and the second row's
// first older tap is the first row's raw row). Each thread takes the same
// four columns of both rows, so the tap weights, the norm scales and the
// barriers are shared, and the two rows' serial sums of squares run side by
// side. The steps and every rounding are front_kernel's, row by row.
template <int ES, int DK, int DV, int REP>
__global__ __launch_bounds__((64 * FrontShape<DK, DV, REP>::W)) void front_pair_kernel(FrontArgs a)
{
#pragma clang fp contract(off)
    using S = FrontShape<DK, DV, REP>;
    constexpr int U = 2;
    __shared__ __align__(16) float ylds[U][S::NH * S::STRIDE];   // conv outputs of the q/k heads
    __shared__ __align__(16) float sqlds[U][S::NH * S::STRIDE];  // their squares
    __shared__ __align__(16) float vlds[U][DV];
    __shared__ float invlds[U][S::NH];

    // rows row0 and row0 + 1 (when below a.rows) of kv group g
    const uint32_t nkv = a.nkv;
    const uint32_t row0 = (blockIdx.x / nkv) * U, g = blockIdx.x % nkv;
    const int tid = threadIdx.x;
    const uint32_t taps = a.taps;
    const uint32_t dq = nkv * REP * DK, dk = nkv * DK, dv = nkv * DV, dcol = dq + dk + dv;
    const bool store = a.k_out == nullptr;
    uint32_t row[U], seq[U], tt[U], pos[U], nt[U];
    bool on[U];
    SeqDev sd[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        on[u] = row0 + u < a.rows;
        row[u] = on[u] ? row0 + u : row0;
        seq[u] = a.row_seq ? a.row_seq[row[u]] : row[u];
        tt[u] = a.row_t ? a.row_t[row[u]] : 0u;
        sd[u] = a.seqs[seq[u]];
        pos[u] = (uint32_t)sd[u].pos + tt[u];
        nt[u] = min(taps, pos[u] + 1u);
    }
    auto hist = [&](int u) __attribute__((always_inline)) {
        return a.hist + ((uint64_t)seq[u] * a.n_layers + a.layer) * taps * dcol;
    };

    // What steps 3 and 4 read (this thread's rotary pairs and norm scales,
    // the page of the stored slot) is requested now, beside the tap loads,
    // so the wave waits on one round of loads rather than three.
    constexpr int NE = (S::NH * S::HALF + 64 * S::W - 1) / (64 * S::W);   // emit elements per thread
    float2 cs_e[U][NE];
    float s1_e[NE], s2_e[NE];
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = tid + n * 64 * S::W;
        const int h = e / S::HALF, i = e % S::HALF;
        if (e < S::NH * S::HALF) {
            const float *sn = a.norm + (h < REP ? 0 : DK);
            s1_e[n] = sn[i];
            s2_e[n] = sn[i + S::HALF];
#pragma unroll
            for (int u = 0; u < U; u++)
                cs_e[u][n] = a.rope[(uint64_t)pos[u] * S::HALF + i];
        }
    }
    int slot[U];
    int32_t page[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        slot[u] = 0;
        page[u] = -1;
        if (store && on[u]) {
            slot[u] = own_slot(sd[u], (int)pos[u], (int)a.pg.window);
            page[u] = a.page_table[(uint64_t)seq[u] * a.pg.pages_per_seq + (slot[u] >> a.pg.log2_page)];
        }
    }

    // 1. tap convolution of this thread's four columns
    const bool active = tid < S::NG;
    const int lc = tid * 4;                      // column within the group
    const float *src;
    uint32_t ld, cc, gc;                         // source row length, column in it, column in dcol
    if (lc < REP * DK) {
        src = a.q; ld = dq; cc = g * REP * DK + lc; gc = cc;
    } else if (lc < REP * DK + DK) {
        src = a.k; ld = dk; cc = g * DK + (lc - REP * DK); gc = dq + cc;
    } else {
        src = a.v; ld = dv; cc = g * DV + (lc - REP * DK - DK); gc = dq + dk + cc;
    }
    if (active) {
        uint32_t ntm = nt[0];                    // taps any of the rows uses
#pragma unroll
        for (int u = 1; u < U; u++)
            ntm = max(ntm, nt[u]);
        float4 w[S::TREG], raw[U], x[U][S::TREG];
#pragma unroll
        for (int j = 0; j < S::TREG; j++)
            if ((uint32_t)j < ntm)
                w[j] = ld4(a.w + (uint64_t)j * dcol + gc);
#pragma unroll
        for (int u = 0; u < U; u++) {
            raw[u] = ld4(src + (uint64_t)row[u] * ld + cc);
#pragma unroll
            for (int j = 1; j < S::TREG; j++) {
                if ((uint32_t)j < nt[u]) {
                    if ((uint32_t)j <= tt[u])
                        x[u][j] = ld4(src + (uint64_t)(row[u] - j) * ld + cc);
                    else
                        x[u][j] = ld4(hist(u) + (uint64_t)((pos[u] - j) % taps) * dcol + gc);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            x[u][0] = raw[u];
#pragma unroll
            for (int j = 0; j < S::TREG; j++)
                if ((uint32_t)j < nt[u])
                    acc4(acc, w[j], x[u][j]);
            for (uint32_t j = S::TREG; j < nt[u]; j++) {
                const float4 wj = ld4(a.w + (uint64_t)j * dcol + gc);
                const float4 xj = j <= tt[u] ? ld4(src + (uint64_t)(row[u] - j) * ld + cc)
                                             : ld4(hist(u) + (uint64_t)((pos[u] - j) % taps) * dcol + gc);
                acc4(acc, wj, xj);
            }
            if (!on[u])
                continue;
            if (a.hist_write)
                *reinterpret_cast<float4 *>(hist(u) + (uint64_t)(pos[u] % taps) * dcol + gc) = raw[u];
            if (lc < (REP + 1) * DK) {
                const int o = (lc / DK) * S::STRIDE + lc % DK;
                *reinterpret_cast<float4 *>(&ylds[u][o]) = acc;
                *reinterpret_cast<float4 *>(&sqlds[u][o]) =
                    make_float4(acc.x * acc.x, acc.y * acc.y, acc.z * acc.z, acc.w * acc.w);
            } else if (store) {
                *reinterpret_cast<float4 *>(&vlds[u][lc - (REP + 1) * DK]) = acc;
            } else {
                *reinterpret_cast<float4 *>(a.v_out + (uint64_t)row[u] * dv + cc) = acc;
            }
        }
    }
    __syncthreads();

    // 2. per-head sum of squares in index order, inverse RMS (one thread per
    // (row, head))
    if (tid < U * S::NH) {
        const int u = tid / S::NH, h = tid % S::NH;
        const float *r = &sqlds[u][h * S::STRIDE];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < DK; i++)
            ss = ss + r[i];
        invlds[u][h] = 1.0f / __builtin_sqrtf(ss / (float)DK + 1e-6f);
    }
    __syncthreads();

    // 3. (1 + s) * x * inv, rotated by the position's (cos, sin)
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (!on[u])
            continue;
#pragma unroll
        for (int n = 0; n < NE; n++) {
            const int e = tid + n * 64 * S::W;
            if (e >= S::NH * S::HALF)
                break;
            const int h = e / S::HALF, i = e % S::HALF;
            const bool is_q = h < REP;
            float *r = &ylds[u][h * S::STRIDE];
            const float iv = invlds[u][h];
            const float x1 = (1.0f + s1_e[n]) * r[i] * iv;
            const float x2 = (1.0f + s2_e[n]) * r[i + S::HALF] * iv;
            const float2 cs = cs_e[u][n];
            const float o1 = x1 * cs.x - x2 * cs.y;
            const float o2 = x2 * cs.x + x1 * cs.y;
            if (is_q) {
                float *qo = a.q_out + (uint64_t)row[u] * dq + (g * REP + h) * DK;
                qo[i] = o1;
                qo[i + S::HALF] = o2;
            } else if (store) {
                r[i] = o1;
                r[i + S::HALF] = o2;
            } else {
                float *ko = a.k_out + (uint64_t)row[u] * dk + g * DK;
                ko[i] = o1;
                ko[i + S::HALF] = o2;
            }
        }
    }
    if (!store)
        return;
    __syncthreads();

    // 4. store each row's k/v rows of kv-head g (wave 0, lane = element)
    if (tid >= 64)
        return;
    const int P = 1 << a.pg.log2_page;
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (page[u] < 0)
            continue;   // a row past the end; the host backs every stored slot
        uint8_t *hb = a.pool + (uint64_t)page[u] * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
        const float kx = tid < DK ? ylds[u][REP * S::STRIDE + tid] : 0.0f;
        const float vx = tid < DV ? vlds[u][tid] : 0.0f;
        store_row<ES>(hb, slot[u] & (P - 1), P, kx, vx, tid, DK, DV);
    }
}

// The same front for every other shape the engine defines (head dims that are
// multiples of 4 up to 64, 1-8 query heads per kv-head), the dims read at run
// time: one 256-thread work-group per (row, kv group), at most 8 * 64 + 64
// + 64 = 640 columns in 160 four-column groups. Same steps and the same order of
// every rounding as front_kernel, so the rows are bit-identical to the
// engine's too.
template <int ES>
__global__ __launch_bounds__(256) void front_rt_kernel(FrontArgs a)
{
#pragma clang fp contract(off)
    constexpr int MAXH = 9, MAXD = 64, STRIDE = MAXD + 4, NT = 256;
    __shared__ __align__(16) float ylds[MAXH * STRIDE];
    __shared__ __align__(16) float sqlds[MAXH * STRIDE];
    __shared__ __align__(16) float vlds[MAXD];
    __shared__ float invlds[MAXH];

    const int DK = (int)a.qk, DV = (int)a.vd, nkv = (int)a.nkv, REP = (int)(a.nh / a.nkv);
    const int NC = REP * DK + DK + DV, NG = NC / 4, NH = REP + 1, HALF = DK / 2;
    const uint32_t row = blockIdx.x / nkv, g = blockIdx.x % nkv;
    const int tid = threadIdx.x;
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const uint32_t t = a.row_t ? a.row_t[row] : 0u;
    const SeqDev sd = a.seqs[seq];
    const uint32_t pos = (uint32_t)sd.pos + t;
    const uint32_t taps = a.taps;
    const uint32_t nt = min(taps, pos + 1u);
    const uint32_t dq = nkv * REP * DK, dk = nkv * DK, dv = nkv * DV, dcol = dq + dk + dv;
    float *hist = a.hist + ((uint64_t)seq * a.n_layers + a.layer) * taps * dcol;
    const bool store = a.k_out == nullptr;

    // 1. tap convolution of this thread's four columns (taps in order)
    const int lc = tid * 4;                      // column within the group
    if (tid < NG) {
        const float *src;
        uint32_t ld, cc, gc;                     // source row length, column in it, column in dcol
        if (lc < REP * DK) {
            src = a.q; ld = dq; cc = g * REP * DK + lc; gc = cc;
        } else if (lc < REP * DK + DK) {
            src = a.k; ld = dk; cc = g * DK + (lc - REP * DK); gc = dq + cc;
        } else {
            src = a.v; ld = dv; cc = g * DV + (lc - REP * DK - DK); gc = dq + dk + cc;
        }
        const float4 raw = ld4(src + (uint64_t)row * ld + cc);
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t j = 0; j < nt; j++) {
            const float4 wj = ld4(a.w + (uint64_t)j * dcol + gc);
            const float4 xj = j == 0 ? raw
                              : j <= t ? ld4(src + (uint64_t)(row - j) * ld + cc)
                                       : ld4(hist + (uint64_t)((pos - j) % taps) * dcol + gc);
            acc4(acc, wj, xj);
        }
        if (a.hist_write)
            *reinterpret_cast<float4 *>(hist + (uint64_t)(pos % taps) * dcol + gc) = raw;
        if (lc < (REP + 1) * DK) {
            const int o = (lc / DK) * STRIDE + lc % DK;
            *reinterpret_cast<float4 *>(ylds + o) = acc;
            *reinterpret_cast<float4 *>(sqlds + o) =
                make_float4(acc.x * acc.x, acc.y * acc.y, acc.z * acc.z, acc.w * acc.w);
        } else if (store) {
            *reinterpret_cast<float4 *>(vlds + (lc - (REP + 1) * DK)) = acc;
        } else {
            *reinterpret_cast<float4 *>(a.v_out + (uint64_t)row * dv + cc) = acc;
        }
    }
    __syncthreads();

    // 2. per-head sum of squares in index order, inverse RMS
    if (tid < NH) {
        const float *r = sqlds + tid * STRIDE;
        float ss = 0.0f;
        for (int i = 0; i < DK; i++)
            ss = ss + r[i];
        invlds[tid] = 1.0f / __builtin_sqrtf(ss / (float)DK + 1e-6f);
    }
    __syncthreads();

    // 3. (1 + s) * x * inv, rotated by the position's (cos, sin)
    const float2 *rope = a.rope + (uint64_t)pos * HALF;
    for (int e = tid; e < NH * HALF; e += NT) {
        const int h = e / HALF, i = e % HALF;
        const bool is_q = h < REP;
        const float *sn = a.norm + (is_q ? 0 : DK);
        float *r = ylds + h * STRIDE;
        const float iv = invlds[h];
        const float x1 = (1.0f + sn[i]) * r[i] * iv;
        const float x2 = (1.0f + sn[i + HALF]) * r[i + HALF] * iv;
        const float2 cs = rope[i];
        const float o1 = x1 * cs.x - x2 * cs.y;
        const float o2 = x2 * cs.x + x1 * cs.y;
        if (is_q) {
            float *qo = a.q_out + (uint64_t)row * dq + (g * REP + h) * DK;
            qo[i] = o1;
            qo[i + HALF] = o2;
        } else if (store) {
            r[i] = o1;
            r[i + HALF] = o2;
        } else {
            float *ko = a.k_out + (uint64_t)row * dk + g * DK;
            ko[i] = o1;
            ko[i + HALF] = o2;
        }
    }
    if (!store)
        return;
    __syncthreads();

    // 4. store this position's k/v rows of kv-head g (wave 0, lane = element)
    if (tid >= 64)
        return;
    const int slot = own_slot(sd, (int)pos, (int)a.pg.window);
    const int32_t page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (slot >> a.pg.log2_page)];
    if (page < 0)
        return;   // the host backs every stored slot; never taken
    const int P = 1 << a.pg.log2_page;
    uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
    const float kx = tid < DK ? ylds[REP * STRIDE + tid] : 0.0f;
    const float vx = tid < DV ? vlds[tid] : 0.0f;
    store_row<ES>(hb, slot & (P - 1), P, kx, vx, tid, DK, DV);
}

// Raw rows of each sequence's last `taps` tokens into their history slots,
// after a multi-token front launch has read the old history.
__global__ __launch_bounds__(256) void hist_tail_kernel(HistTailArgs a)
{
    const uint32_t row = blockIdx.x;
    const uint32_t t = a.row_t[row], n = a.row_n[row];
    if (t + a.taps < n)
        return;
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const uint32_t pos = (uint32_t)a.seqs[seq].pos + t;
    const uint32_t dcol = a.dq + a.dk + a.dv;
    float *h = a.hist + (((uint64_t)seq * a.n_layers + a.layer) * a.taps + pos % a.taps) * dcol;
    for (uint32_t c = threadIdx.x; c < dcol; c += 256) {
        float x;
        if (c < a.dq)
            x = a.q[(uint64_t)row * a.dq + c];
        else if (c < a.dq + a.dk)
            x = a.k[(uint64_t)row * a.dk + (c - a.dq)];
        else
            x = a.v[(uint64_t)row * a.dv + (c - a.dq - a.dk)];
        h[c] = x;
    }
}

// Whole-block history copies / clears: grid.y = op, grid.x strides the block.
__global__ __launch_bounds__(256) void hist_ops_kernel(const HistOp *ops, uint64_t block_floats)
{
    const HistOp op = ops[blockIdx.y];
    const uint64_t n4 = block_floats / 4;
    float4 *d = reinterpret_cast<float4 *>(op.dst);
    const float4 *s = reinterpret_cast<const float4 *>(op.src);
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * 256)
        d[i] = s ? s[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// Rows per work-group: 2 (front_pair_kernel) for launches of several tokens per
// sequence (those that leave the history writes to hist_tail_kernel; rows t,
// t + 1 of one sequence, the second row's first older tap being the first
// row's raw row) of at least FRONT_PAIR_UNITS (row, kv group) units, 1
// otherwise. Block prefill, 49,787 rows x 2 kv groups: 0.95 against
// 1.08 ms per 8-layer pass; the 4096-row decode fronts (one row per sequence)
// were slower with 2 (0.0332 against 0.0293 ms, 8 kv groups).
constexpr uint64_t FRONT_PAIR_UNITS = 4096;

hipError_t launch_front(const Geo &g, const FrontArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    const bool pair = !a.hist_write && (uint64_t)a.rows * a.nkv >= FRONT_PAIR_UNITS;
    const dim3 grid(a.rows * a.nkv), grid2((a.rows + 1) / 2 * a.nkv);
#define X(ES, DK, DV, REP)                                                                      \
    if ((g.kv_f16 ? 2 : 1) == ES && g.dk == DK && g.dv == DV && g.rep == REP) {                \
        if (pair)                                                                               \
            hipLaunchKernelGGL((front_pair_kernel<ES, DK, DV, REP>), grid2,                     \
                               dim3((64 * FrontShape<DK, DV, REP>::W)), 0, s, a);               \
        else                                                                                    \
            hipLaunchKernelGGL((front_kernel<ES, DK, DV, REP>), grid,                           \
                               dim3((64 * FrontShape<DK, DV, REP>::W)), 0, s, a);               \
        return hipGetLastError();                                                               \
    }
    NDA_FOR_GEOMETRIES(X)
#undef X
    if (!geometry_supported(g))
        return hipErrorNotSupported;
    if (g.kv_f16)
        hipLaunchKernelGGL((front_rt_kernel<2>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((front_rt_kernel<1>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_hist_tail(const HistTailArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    hipLaunchKernelGGL(hist_tail_kernel, dim3(a.rows), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_hist_ops(const HistOp *d_ops, uint32_t n_ops, uint64_t block_floats, hipStream_t s)
{
    if (n_ops == 0)
        return hipSuccess;
    const uint64_t n4 = block_floats / 4;
    const unsigned gx = (unsigned)std::min<uint64_t>((n4 + 255) / 256, 64);
    hipLaunchKernelGGL(hist_ops_kernel, dim3(gx, n_ops), dim3(256), 0, s, d_ops, block_floats);
    return hipGetLastError();
}

} // namespace nda
