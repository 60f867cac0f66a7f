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
// is reused by all rows. The GEMM decodes each 64-output x group tile of
// codes once per work-group into LDS as fp32 cb * norm, stages the matching
// 64-row xh tile beside it, and accumulates on v_mfma_f32_32x32x2_f32 (fp32
// products and sums: the result is the engine's up to fp32 reassociation).
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
constexpr int CQ_KT = 64;     // reduction columns per LDS tile (divides every group size used)

// LDS row of one tile, k-permuted so that MFMA step s of lane half h reads
// column 2s + h at [h*KT/2 + s]: four steps are one 16-byte read. +4 floats
// of pad per row keep rows 16-byte aligned and spread over the banks.
constexpr int CQ_KS = CQ_KT + 4;

__device__ __forceinline__ int cq_perm(int k) { return (k & 1) * (CQ_KT / 2) + (k >> 1); }

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

__global__ __launch_bounds__(256) void cq_gemm_kernel(CqGemmArgs a)
{
    __shared__ __attribute__((aligned(16))) float Xs[CQ_MT][CQ_KS];
    __shared__ __attribute__((aligned(16))) float Ws[CQ_NT][CQ_KS];
    __shared__ float cbs[16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 31, lh = lane >> 5;
    const uint32_t r0 = blockIdx.x * CQ_MT, o0 = blockIdx.y * CQ_NT;
    const int wr = (wave & 1) * 32, wo = (wave >> 1) * 32;     // this wave's 32 x 32 block

    if (tid < (1 << a.bits))
        cbs[tid] = a.cb[tid];

    float16v acc = {};
    for (uint32_t k0 = 0; k0 < a.in_pad; k0 += CQ_KT) {
        __syncthreads();      // previous tile's readers done (and cbs visible on the first pass)
        // xh tile: 64 rows x 64 columns, float4 per thread per step
        for (int c = tid; c < CQ_MT * CQ_KT / 4; c += 256) {
            const int rr = c / (CQ_KT / 4), kk = (c % (CQ_KT / 4)) * 4;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r0 + rr < a.rows && k0 + kk < a.in_pad)       // in_pad is a multiple of 4
                v = *reinterpret_cast<const float4 *>(a.xh + (uint64_t)(r0 + rr) * a.in_pad + k0 + kk);
            Xs[rr][cq_perm(kk + 0)] = v.x;
            Xs[rr][cq_perm(kk + 1)] = v.y;
            Xs[rr][cq_perm(kk + 2)] = v.z;
            Xs[rr][cq_perm(kk + 3)] = v.w;
        }
        // weight tile: decode codes, * the group norm
        for (int c = tid; c < CQ_NT * CQ_KT; c += 256) {
            const int oo = c / CQ_KT, kk = c % CQ_KT;
            float w = 0.0f;
            const uint32_t k = k0 + kk;
            if (o0 + oo < a.out && k < a.in_pad) {
                const uint8_t *row = a.packed + (uint64_t)(o0 + oo) * a.rowbytes;
                const uint16_t nb = a.norms[(uint64_t)(o0 + oo) * a.ngroup + k / a.group];
                w = cbs[cq_code(row, k, a.bits)] * half_bits_to_float(nb);
            }
            Ws[oo][cq_perm(kk)] = w;
        }
        __syncthreads();
        // 32 MFMA steps of K = 2: A = xh rows (lane: row ln, column 2s + lh),
        // B = W^T (lane: output ln, column 2s + lh)
        const float *xa = &Xs[wr + ln][lh * (CQ_KT / 2)];
        const float *wb = &Ws[wo + ln][lh * (CQ_KT / 2)];
#pragma unroll
        for (int s4 = 0; s4 < CQ_KT / 2; s4 += 4) {
            const float4v xv = *reinterpret_cast<const float4v *>(xa + s4);
            const float4v wv = *reinterpret_cast<const float4v *>(wb + s4);
#pragma unroll
            for (int e = 0; e < 4; e++)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[e], wv[e], acc, 0, 0, 0);
        }
    }
    // C layout: lane holds output column ln, rows 8*(i/4) + 4*lh + (i%4)
    const uint32_t oc = o0 + wo + ln;
    if (oc >= a.out)
        return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t rr = r0 + wr + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (rr < a.rows)
            a.y[(uint64_t)rr * a.out + oc] = acc[i];
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
    if (a.rows == 0 || a.out == 0)
        return hipSuccess;
    const dim3 grid((a.rows + CQ_MT - 1) / CQ_MT, (a.out + CQ_NT - 1) / CQ_NT);
    hipLaunchKernelGGL(cq_gemm_kernel, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

} // namespace nda
