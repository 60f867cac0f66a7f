// nda_cq.hip - CQ projections on gfx950: the engine's codebook-quantised
// matvecs (engine/src/nd_quant.c, engine/include/nd_quant.h) for many rows
// at once.
//
// A CQ tensor [out][in] stores per group of `group` weights a `bits`-wide
// codebook index per weight (an LSB-first bitstream per row) and one fp16
// norm per (row, group); w_group = (cb[idx] * norm) @ H with H the
// orthonormal Walsh-Hadamard matrix. As in the engine, the activation is
// transformed instead of the weights:
//
//   cq_prepare_kernel   xh = per-group H x (zero-padded to in_pad), the
//                       engine's butterfly order and rescale (nd_fwht +
//                       fw_scale, :36-65, :99-116), so xh is bit-identical
//   cq_gemm_kernel      y[r][o] = sum_k cb[idx[o][k]] * norm[o][k/group] *
//                       xh[r][k] over all rows r of the batch
//
// The engine runs one row against the weights (a GEMV that streams the
// compressed weights); a batch of rows makes it a GEMM in which every weight
// is reused by all rows. Per 64-column step a work-group decodes a 64-output
// tile of codes into LDS as fp32 cb * norm, stages the matching 64-row xh
// tile beside it (the next step's loads in flight during this step's MFMAs),
// and accumulates on v_mfma_f32_32x32x2_f32 (fp32 products and sums: the
// result is the engine's up to fp32 reassociation).
#include "nda_device.h"

#include <algorithm>

namespace nda {

// ---------------------------------------------------------------- prepare

// One work-group per row: the row's in_pad values in LDS, log2(group)
// butterfly stages (stage len pairs j and j+len inside each block of 2*len,
// out = (a + b, a - b) with a the lower element, as nd_fwht), then * scale.
__global__ __launch_bounds__(256) void cq_prepare_kernel(CqPrepArgs a)
{
    extern __shared__ float xs[];
    const uint32_t row = blockIdx.x;
    const float *x = a.x + (uint64_t)row * a.in;
    for (uint32_t i = threadIdx.x; i < a.in_pad; i += 256)
        xs[i] = i < a.in ? x[i] : 0.0f;
    __syncthreads();
    for (uint32_t len = 1; len < a.group; len <<= 1) {
        for (uint32_t p = threadIdx.x; p < a.in_pad / 2; p += 256) {
            const uint32_t j = (p / len) * (2 * len) + p % len;
            const float u = xs[j], v = xs[j + len];
            xs[j] = u + v;
            xs[j + len] = u - v;
        }
        __syncthreads();
    }
    float *xh = a.xh + (uint64_t)row * a.in_pad;
    for (uint32_t i = threadIdx.x; i < a.in_pad; i += 256)
        xh[i] = xs[i] * a.scale;
}

// ------------------------------------------------------------------- GEMM

typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int CQ_MT = 64;     // rows per work-group
constexpr int CQ_NT = 64;     // outputs per work-group
constexpr int CQ_KT = 64;     // reduction columns per LDS tile
constexpr int CQ_KS = CQ_KT + 4;   // LDS row: +4 floats keep rows 16-byte aligned, banks spread

// Index k of one row's bitstream (bits 2, 3 or 4): at most two bytes.
__device__ __forceinline__ uint32_t cq_code(const uint8_t *row, uint32_t k, uint32_t bits)
{
    const uint32_t b = k * bits, byt = b >> 3, sh = b & 7u;
    uint32_t w = row[byt];
    if (sh + bits > 8)
        w |= (uint32_t)row[byt + 1] << 8;
    return (w >> sh) & ((1u << bits) - 1u);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// One thread's share of a tile in flight: 4 float4 of xh (rows tid/16 + 16 i,
// columns 4 (tid%16)..) and the 16 codes of one (output, 16-column) slice
// with its group norm.
struct CqStage {
    float4 x[4];
    uint32_t code[2];     // 16 codes: one word at 2 bits, two at 4 bits
    uint16_t norm;
};

// WORDS: the 16 codes of a slice are one (2-bit) or two (4-bit) aligned
// 32-bit words; otherwise (3 bits, or rows not 4-byte aligned) they are
// read field by field at decode time.
template <bool WORDS>
__global__ __launch_bounds__(256) void cq_gemm_kernel(CqGemmArgs a)
{
    __shared__ __attribute__((aligned(16))) float Xs[CQ_MT][CQ_KS];
    __shared__ __attribute__((aligned(16))) float Ws[CQ_NT][CQ_KS];
    __shared__ float cbs[16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 31, lh = lane >> 5;
    // which tensor this output tile belongs to
    uint32_t ti = 0;
    while (ti + 1 < a.nt && blockIdx.y >= a.tile0[ti + 1])
        ti++;
    const uint32_t out = a.out[ti];
    const uint8_t *packed = a.packed[ti];
    const uint16_t *norms = a.norms[ti];
    float *y = a.y[ti];
    const uint32_t r0 = blockIdx.x * CQ_MT, o0 = (blockIdx.y - a.tile0[ti]) * CQ_NT;
    const int wr = (wave & 1) * 32, wo = (wave >> 1) * 32;     // this wave's 32 x 32 block
    const int xr = tid >> 4, xc = (tid & 15) * 4;               // xh: rows xr + 16 i, columns xc..xc+3
    const int wrow = tid >> 2, wc = (tid & 3) * 16;             // weights: output wrow, columns wc..wc+15
    const bool wvalid = o0 + wrow < out;
    const uint8_t *wrp = packed + (uint64_t)(o0 + wrow) * a.rowbytes;

    if (tid < (1 << a.bits))
        cbs[tid] = a.cb[ti][tid];

    auto load = [&](uint32_t k0, CqStage &sg) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t r = r0 + xr + 16 * i;
            sg.x[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r < a.rows && k0 + xc < a.in_pad)          // in_pad is a multiple of 8
                sg.x[i] = *reinterpret_cast<const float4 *>(a.xh + (uint64_t)r * a.in_pad + k0 + xc);
        }
        const uint32_t k = k0 + wc;
        sg.code[0] = sg.code[1] = 0;
        sg.norm = 0;
        if (wvalid && k < a.in_pad) {
            sg.norm = norms[(uint64_t)(o0 + wrow) * a.ngroup + k / a.group];
            if constexpr (WORDS) {
                const uint32_t *wp = reinterpret_cast<const uint32_t *>(wrp + (k * a.bits >> 3));
                sg.code[0] = wp[0];
                if (a.bits == 4)
                    sg.code[1] = wp[1];
            }
        }
    };
    auto store = [&](uint32_t k0, const CqStage &sg) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<float4 *>(&Xs[xr + 16 * i][xc]) = sg.x[i];
        const float nf = half_bits_to_float(sg.norm);
        float w[16];
        const uint32_t k = k0 + wc;
        const uint32_t lim = a.in_pad - min(k, a.in_pad);   // columns of this slice inside the row
#pragma unroll
        for (int e = 0; e < 16; e++) {
            uint32_t c;
            if constexpr (WORDS)
                c = a.bits == 2 ? (sg.code[0] >> (2 * e)) & 3u : (sg.code[e >> 3] >> (4 * (e & 7))) & 15u;
            else
                c = wvalid && (uint32_t)e < lim ? cq_code(wrp, k + e, a.bits) : 0u;
            w[e] = cbs[c] * nf;
        }
#pragma unroll
        for (int e = 0; e < 16; e += 4)
            *reinterpret_cast<float4 *>(&Ws[wrow][wc + e]) = make_float4(w[e], w[e + 1], w[e + 2], w[e + 3]);
    };

    float16v acc = {};
    CqStage sg;
    load(0, sg);
    __syncthreads();          // cbs visible
    for (uint32_t k0 = 0; k0 < a.in_pad; k0 += CQ_KT) {
        store(k0, sg);
        __syncthreads();
        if (k0 + CQ_KT < a.in_pad)
            load(k0 + CQ_KT, sg);       // lands during this tile's MFMAs
        // 32 MFMA steps of K = 2. Step 4j+e takes column 8j+e in lane half 0
        // and 8j+4+e in lane half 1, for A (xh rows) and B (W^T) alike, so a
        // lane reads four steps' operands as one 16-byte word.
        const float *xa = &Xs[wr + ln][4 * lh];
        const float *wb = &Ws[wo + ln][4 * lh];
#pragma unroll
        for (int j = 0; j < CQ_KT / 8; j++) {
            const float4v xv = *reinterpret_cast<const float4v *>(xa + 8 * j);
            const float4v wv = *reinterpret_cast<const float4v *>(wb + 8 * j);
#pragma unroll
            for (int e = 0; e < 4; e++)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[e], wv[e], acc, 0, 0, 0);
        }
        __syncthreads();      // readers done before the next store
    }
    // C layout: lane holds output column ln, rows 8*(i/4) + 4*lh + (i%4)
    const uint32_t oc = o0 + wo + ln;
    if (oc >= out)
        return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t rr = r0 + wr + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (rr < a.rows)
            y[(uint64_t)rr * out + oc] = acc[i];
    }
}

hipError_t launch_cq_prepare(const CqPrepArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    hipLaunchKernelGGL(cq_prepare_kernel, dim3(a.rows), dim3(256), a.in_pad * sizeof(float), s, a);
    return hipGetLastError();
}

hipError_t launch_cq_gemm(const CqGemmArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.nt == 0 || a.tile0[a.nt] == 0)
        return hipSuccess;
    const dim3 grid((a.rows + CQ_MT - 1) / CQ_MT, a.tile0[a.nt]);
    const bool words = (a.bits == 2 || a.bits == 4) && a.rowbytes % 4 == 0;
    if (words)
        hipLaunchKernelGGL(cq_gemm_kernel<true>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(cq_gemm_kernel<false>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

} // namespace nda
