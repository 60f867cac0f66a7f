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
// One work-group per row (one token of one sequence) covers every column of
// q, k and v: the convolution is one column per thread, the per-head sums of
// squares one head per thread (a sequential walk, the reference's order),
// the emit one (head, rotary pair) per thread. Store mode then writes the k/v
// rows into the KV pages exactly as the append kernel does (int8 with the
// engine's Markstein store, or fp16), so the decode launch that follows reads
// them from the cache.
//
// Every multiply and add rounds on its own (no contraction) and divide / sqrt
// are correctly rounded, so the results are bit-identical to the engine's
// host build, and so are the int8 codes computed from them.
#include "nda_device.h"

namespace nda {

namespace {

// LDS layout: the q and k heads' convolution outputs, one row of qk+1 floats
// per head (the pad keeps the one-head-per-thread column walk free of bank
// conflicts), then v, then one inverse RMS per q/k head.
struct FrontLds {
    uint32_t stride, nqk, v_off, inv_off, total;
};

__host__ __device__ inline FrontLds front_lds(uint32_t nh, uint32_t nkv, uint32_t qk, uint32_t vd)
{
    FrontLds l;
    l.stride = qk + 1;
    l.nqk = nh + nkv;
    l.v_off = l.nqk * l.stride;
    l.inv_off = l.v_off + nkv * vd;
    l.total = l.inv_off + l.nqk;
    return l;
}

} // namespace

template <int ES, int DK, int DV>
__global__ __launch_bounds__(256) void front_kernel(FrontArgs a)
{
#pragma clang fp contract(off)
    extern __shared__ float lds[];
    const uint32_t row = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const uint32_t t = a.row_t ? a.row_t[row] : 0u;
    const SeqDev sd = a.seqs[seq];
    const uint32_t pos = (uint32_t)sd.pos + t;
    const uint32_t taps = a.taps;
    const uint32_t nt = min(taps, pos + 1u);
    const uint32_t nh = a.nh, nkv = a.nkv;
    const uint32_t dq = nh * DK, dk = nkv * DK, dv = nkv * DV, dcol = dq + dk + dv;
    const FrontLds L = front_lds(nh, nkv, DK, DV);
    float *hist = a.hist + ((uint64_t)seq * a.n_layers + a.layer) * taps * dcol;
    const bool store = a.k_out == nullptr;

    // 1. tap convolution, one column per thread
    for (uint32_t c = tid; c < dcol; c += 256) {
        const float *src;
        uint32_t cc, ld;
        if (c < dq) {
            src = a.q; cc = c; ld = dq;
        } else if (c < dq + dk) {
            src = a.k; cc = c - dq; ld = dk;
        } else {
            src = a.v; cc = c - dq - dk; ld = dv;
        }
        const float raw = src[(uint64_t)row * ld + cc];
        float acc = 0.0f;
        for (uint32_t j = 0; j < nt; j++) {
            float x;
            if (j == 0)
                x = raw;
            else if (j <= t)
                x = src[(uint64_t)(row - j) * ld + cc];
            else
                x = hist[(uint64_t)((pos - j) % taps) * dcol + c];
            acc = acc + a.w[(uint64_t)j * dcol + c] * x;
        }
        if (a.hist_write)
            hist[(uint64_t)(pos % taps) * dcol + c] = raw;
        if (c < dq + dk) {
            lds[(c / DK) * L.stride + (c % DK)] = acc;
        } else if (store) {
            lds[L.v_off + cc] = acc;
        } else {
            a.v_out[(uint64_t)row * dv + cc] = acc;
        }
    }
    __syncthreads();

    // 2. per-head sum of squares in index order, inverse RMS
    for (uint32_t h = tid; h < L.nqk; h += 256) {
        const float *r = lds + h * L.stride;
        float ss = 0.0f;
#pragma unroll 8
        for (uint32_t i = 0; i < DK; i++)
            ss = ss + r[i] * r[i];
        lds[L.inv_off + h] = 1.0f / __builtin_sqrtf(ss / (float)DK + 1e-6f);
    }
    __syncthreads();

    // 3. (1 + s) * x * inv, rotated by the position's (cos, sin)
    constexpr uint32_t HALF = DK / 2;
    const float2 *rope = a.rope + (uint64_t)pos * HALF;
    for (uint32_t e = tid; e < L.nqk * HALF; e += 256) {
        const uint32_t h = e / HALF, i = e % HALF;
        const bool is_q = h < nh;
        const float *s = a.norm + (is_q ? 0 : DK);
        float *r = lds + h * L.stride;
        const float iv = lds[L.inv_off + h];
        const float x1 = (1.0f + s[i]) * r[i] * iv;
        const float x2 = (1.0f + s[i + HALF]) * r[i + HALF] * iv;
        const float2 cs = rope[i];
        const float o1 = x1 * cs.x - x2 * cs.y;
        const float o2 = x2 * cs.x + x1 * cs.y;
        if (is_q) {
            float *qo = a.q_out + (uint64_t)row * dq + h * DK;
            qo[i] = o1;
            qo[i + HALF] = o2;
        } else if (store) {
            r[i] = o1;
            r[i + HALF] = o2;
        } else {
            float *ko = a.k_out + (uint64_t)row * dk + (h - nh) * DK;
            ko[i] = o1;
            ko[i + HALF] = o2;
        }
    }
    if (!store)
        return;
    __syncthreads();

    // 4. store this position's k/v rows (one wave per kv-head)
    const int slot = own_slot(sd, (int)pos, (int)a.pg.window);
    const int P = 1 << a.pg.log2_page;
    const int32_t page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (slot >> a.pg.log2_page)];
    if (page < 0)
        return;   // the host backs every stored slot; never taken
    const int off = slot & (P - 1);
    const int lane = tid & 63;
    for (uint32_t g = tid >> 6; g < nkv; g += 4) {
        uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
        const float kx = lane < DK ? lds[(nh + g) * L.stride + lane] : 0.0f;
        const float vx = lane < DV ? lds[L.v_off + g * DV + lane] : 0.0f;
        store_row<ES, DK, DV>(hb, off, P, kx, vx, lane);
    }
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

size_t front_lds_bytes(const FrontArgs &a)
{
    return (size_t)front_lds(a.nh, a.nkv, a.qk, a.vd).total * sizeof(float);
}

#define NDA_FRONT_SHAPES(X) X(2, 64, 64) X(2, 48, 64) X(1, 64, 64) X(1, 48, 64)

hipError_t launch_front(const Geo &g, const FrontArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    const size_t lds = front_lds_bytes(a);
#define X(ES, DK, DV)                                                                          \
    if ((g.kv_f16 ? 2 : 1) == ES && g.dk == DK && g.dv == DV) {                               \
        hipLaunchKernelGGL((front_kernel<ES, DK, DV>), dim3(a.rows), dim3(256), lds, s, a);    \
        return hipGetLastError();                                                              \
    }
    NDA_FRONT_SHAPES(X)
#undef X
    return hipErrorNotSupported;
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
