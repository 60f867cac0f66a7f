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
#include <float.h>

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
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// ------------------------------------------------ split-precision path
//
// For 2-bit tensors with group >= 32 the GEMM runs on fp16 MFMA
// (v_mfma_f32_32x32x16_f16, 16x the fp32 rate) with each fp32 operand
// carried as a pair of fp16 values:
//   xh * 2^rexp[r]  = xa + xb     per row, from the split prepare
//   cb[c] * 2^ecb   = ca + cb'    per tensor, its four codebook entries
//   sum_k w x  ~  sum_k (ca xa + ca xb + cb' xa)   (cb' xb, 2^-22 relative, dropped)
// Products and sums are fp32 inside the MFMA. A group's sum is scaled by
// its norm into the running total, and the total by 2^-(rexp + ecb) at the
// end. The powers of two put each row's and the codebook's largest |value|
// in [2^14, 2^15), so every fp16 part is a normal number with its full 11
// bits: the pairs hold 22 significant bits, and the result stays within
// fp32 reassociation of the engine's matvec (a few 2^-22 of sum |w x|).
//
// The split rows are stored in the order the MFMA reads them: per block of
// 32 rows and 16 columns, per plane (a, b), the 64 lanes' 16-byte operands
// (lane = row % 32 + 32 * (column % 16 / 8), 8 consecutive columns), so one
// wave loads an operand as one contiguous 1 KiB.

__device__ __forceinline__ uint64_t split_index(uint32_t row, uint32_t col, uint32_t nkb, int plane)
{
    const uint32_t rb = row >> 5, kb = col >> 4, lane = (row & 31) + ((col >> 3) & 1) * 32;
    return ((((uint64_t)rb * nkb + kb) * 2 + plane) * 64 + lane) * 8 + (col & 7);
}

// One wave per row, up to four rows per work-group (as many as fit 64 KiB
// of LDS): the wave's row in LDS, the butterfly stages of cq_prepare_kernel
// (same pairs, same order, so the values are the engine's bit for bit)
// separated by wave-level barriers only, the row maximum by shuffles.

__global__ __launch_bounds__(256) void cq_prepare_split_kernel(CqPrepSplitArgs a)
{
    extern __shared__ float xsh[];      // CQ_PREP_ROWS rows of in_pad values
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * a.rpw + wave;
    if ((uint32_t)wave >= a.rpw || row >= a.rows)
        return;                         // no block barrier below: the other waves go on
    float *xs = xsh + (size_t)wave * a.in_pad;
    const float *x = a.x + (uint64_t)row * a.in;
    for (uint32_t i = lane; i < a.in_pad; i += 64)
        xs[i] = i < a.in ? x[i] : 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (uint32_t len = 1; len < a.group; len <<= 1) {
        for (uint32_t p = lane; p < a.in_pad / 2; p += 64) {
            const uint32_t j = (p / len) * (2 * len) + p % len;
            const float u = xs[j], v = xs[j + len];
            xs[j] = u + v;
            xs[j + len] = u - v;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float m = 0.0f;
    for (uint32_t i = lane; i < a.in_pad; i += 64) {
        const float v = xs[i] * a.scale;        // the engine's prepared value
        xs[i] = v;
        m = fmaxf(m, fabsf(v));
    }
    m = wave_max(m);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int e = 0, sh = 0;
    if (m > 0.0f && m <= FLT_MAX) {
        (void)frexpf(m, &e);
        sh = 15 - e;                            // m * 2^sh in [2^14, 2^15)
    }
    // eight consecutive columns per lane: one 16-byte store per plane
    const uint32_t nkb = a.in_pad / 16;
    for (uint32_t c0 = 8 * lane; c0 < a.in_pad; c0 += 8 * 64) {
        _Float16 h8[8], l8[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float v = ldexpf(xs[c0 + s], sh);
            asm volatile("" : "+v"(v));         // both halves from this one value
            h8[s] = (_Float16)v;
            l8[s] = (_Float16)(v - (float)h8[s]);
        }
        *reinterpret_cast<half8 *>(a.xs + split_index(row, c0, nkb, 0)) =
            half8{h8[0], h8[1], h8[2], h8[3], h8[4], h8[5], h8[6], h8[7]};
        *reinterpret_cast<half8 *>(a.xs + split_index(row, c0, nkb, 1)) =
            half8{l8[0], l8[1], l8[2], l8[3], l8[4], l8[5], l8[6], l8[7]};
    }
    if (lane == 0)
        a.rexp[row] = sh;
}

// Register form for rows of up to 1536 columns and groups of at least 64:
// one wave per row, lane l holding columns 512 h + 8 l .. +7 (h < 3). The
// butterfly stages are the engine's (the same pairs, a + b and a - b, stage
// by stage): len < 8 inside a lane, 8 <= len < 512 between lanes l and
// l ^ (len / 8) (the upper lane's a - b as fmaf(-1, b, a), one rounding of
// the same exact difference), len >= 512 between a lane's column blocks.
// The values are the engine's bit for bit. A work-group is 8 consecutive
// rows (8 waves); their 16-byte operand slots meet in LDS, and each 128-byte
// line of the split rows (8 rows x one slot) is then written whole.
constexpr int CQ_REG_COLS = 1536;

__global__ __launch_bounds__(512) void cq_prepare_split_reg_kernel(CqPrepSplitArgs a)
{
    __shared__ __attribute__((aligned(16))) uint4 T[2][CQ_REG_COLS / 8][9];   // [plane][slot][row of 8 + pad]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.x * 8, row = row0 + wave;
    const bool live = row < a.rows;
    const float *x = a.x + (uint64_t)(live ? row : 0) * a.in;
    float v[3][8];
    const bool vec = (a.in & 3) == 0;                  // rows 16-byte aligned
#pragma unroll
    for (int h = 0; h < 3; h++) {
        const uint32_t i0 = 512 * h + 8 * lane;
        if (vec && live && i0 + 8 <= a.in) {           // two 16-byte loads
            const float4 p = *reinterpret_cast<const float4 *>(x + i0);
            const float4 q = *reinterpret_cast<const float4 *>(x + i0 + 4);
            v[h][0] = p.x; v[h][1] = p.y; v[h][2] = p.z; v[h][3] = p.w;
            v[h][4] = q.x; v[h][5] = q.y; v[h][6] = q.z; v[h][7] = q.w;
        } else {
#pragma unroll
            for (int s = 0; s < 8; s++)
                v[h][s] = live && i0 + s < a.in ? x[i0 + s] : 0.0f;
        }
    }
    const int nh = (int)((a.in_pad + 511) / 512);       // column blocks in use (<= 3)
    for (uint32_t len = 1; len < a.group; len <<= 1) {
        if (len < 8) {
#pragma unroll
            for (int h = 0; h < 3; h++)
                if (h < nh)
#pragma unroll
                for (int s = 0; s < 8; s++)
                    if ((s & len) == 0) {
                        const float u = v[h][s], w = v[h][s + len];
                        v[h][s] = u + w;
                        v[h][s + len] = u - w;
                    }
        } else if (len < 512) {
            const int m = (int)(len >> 3);
            const float sg = (lane & m) ? -1.0f : 1.0f;
#pragma unroll
            for (int h = 0; h < 3; h++)
                if (h < nh)
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    const float w = __shfl_xor(v[h][s], m, 64);
                    v[h][s] = fmaf(sg, v[h][s], w);     // lower lane: v + w; upper: w - v
                }
        } else {
            const int m = (int)(len >> 9);
#pragma unroll
            for (int h = 0; h < 3; h++)
                if ((h & m) == 0)
#pragma unroll
                    for (int s = 0; s < 8; s++) {
                        const float u = v[h][s], w = v[h + m][s];
                        v[h][s] = u + w;
                        v[h + m][s] = u - w;
                    }
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int h = 0; h < 3; h++)
#pragma unroll
        for (int s = 0; s < 8; s++) {
            v[h][s] *= a.scale;                         // the engine's prepared value
            if (512 * h + 8 * lane < a.in_pad)
                mx = fmaxf(mx, fabsf(v[h][s]));
        }
    mx = wave_max(mx);
    int e = 0, sh = 0;
    if (mx > 0.0f && mx <= FLT_MAX) {
        (void)frexpf(mx, &e);
        sh = 15 - e;                                   // mx * 2^sh in [2^14, 2^15)
    }
    // this row's operand slots into LDS, then whole lines out
#pragma unroll
    for (int h = 0; h < 3; h++) {
        const uint32_t c = 64 * h + lane;              // slot: columns 8c .. 8c + 7
        if (8 * c >= a.in_pad)
            continue;
        _Float16 h8[8], l8[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float y = ldexpf(v[h][s], sh);
            asm volatile("" : "+v"(y));                // both halves from this one value
            h8[s] = (_Float16)y;
            l8[s] = (_Float16)(y - (float)h8[s]);
        }
        T[0][c][wave] = __builtin_bit_cast(uint4, half8{h8[0], h8[1], h8[2], h8[3], h8[4], h8[5], h8[6], h8[7]});
        T[1][c][wave] = __builtin_bit_cast(uint4, half8{l8[0], l8[1], l8[2], l8[3], l8[4], l8[5], l8[6], l8[7]});
    }
    if (live && lane == 0)
        a.rexp[row] = sh;
    __syncthreads();
    // 8 rows' slot c of a plane is one 128-byte line (lanes row0 % 32 ..
    // +7 of one operand): thread t writes row t % 8 of line t / 8
    const uint32_t nslot = a.in_pad / 8, nkb = a.in_pad / 16;
    for (uint32_t u = threadIdx.x; u < 2 * nslot * 8; u += 512) {
        const uint32_t r = u & 7, c = (u >> 3) % nslot, p = (u >> 3) / nslot;
        *reinterpret_cast<uint4 *>(a.xs + split_index(row0 + r, 8 * c, nkb, (int)p)) = T[p][c][r];
    }
}

constexpr int CS_KT = 32;           // reduction columns per step: two MFMA k-blocks

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Work-group = 128 rows x 128 outputs of one tensor, 4 waves of 64 x 64
// (2 x 2 blocks of 32 x 32) that share only the code tables: each wave loads
// its X operands straight from the split rows (one step ahead, in two
// register sets used in turn) and decodes its W operands from the codes
// through two 256-entry tables (one byte = four 2-bit codes -> their four
// fp16 a parts, and their four b parts). No barrier inside the loop. Loads
// for rows or outputs past the end read row 0 instead (in bounds); what
// they feed lands only in rows or columns that are never stored.
template <int OB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OB >= 2 ? 2 : 3)))
void cq_gemm_split_kernel(CqSplitArgs a)
{
    __shared__ u32x2 luta[256], lutb[256];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 31, jh = lane >> 5;
    // XCD-aware order: work-group w runs on XCD w % 8; consecutive work
    // items are the output tiles of one row tile, which read the same X
    // rows, so they go to one XCD and share its L2. The grid is padded to a
    // multiple of 8.
    const uint32_t nwg = gridDim.x, item = (blockIdx.x % 8u) * (nwg / 8u) + blockIdx.x / 8u;
    const uint32_t ntiles = a.tile0[a.nt];
    const uint32_t rtile = item / ntiles, otile = item % ntiles;
    if (rtile * CQ_SPLIT_MT >= a.rows)
        return;                         // padding
    uint32_t ti = 0;
    while (ti + 1 < a.nt && otile >= a.tile0[ti + 1])
        ti++;
    const uint32_t out = a.out[ti];
    float *y = a.y[ti];
    const uint32_t r0 = rtile * CQ_SPLIT_MT, o0 = (otile - a.tile0[ti]) * (64 * OB);
    const int wr = (wave & 1) * 64, wo = (wave >> 1) * 32 * OB;

    // the codebook as fp16 pairs, scaled so its largest |entry| is in [2^14, 2^15)
    const float *cbp = a.cb[ti];
    const float cbv[4] = {cbp[0], cbp[1], cbp[2], cbp[3]};
    const float cm = fmaxf(fmaxf(fabsf(cbv[0]), fabsf(cbv[1])), fmaxf(fabsf(cbv[2]), fabsf(cbv[3])));
    int ecb = 0;
    if (cm > 0.0f && cm <= FLT_MAX) {
        int e;
        (void)frexpf(cm, &e);
        ecb = 15 - e;
    }
    {
        uint32_t hw[2] = {0u, 0u}, lw[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = (tid >> (2 * j)) & 3;
            float v = ldexpf(c == 0 ? cbv[0] : c == 1 ? cbv[1] : c == 2 ? cbv[2] : cbv[3], ecb);
            asm volatile("" : "+v"(v));
            const _Float16 h = (_Float16)v, l = (_Float16)(v - (float)h);
            hw[j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, h) << (16 * (j & 1));
            lw[j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, l) << (16 * (j & 1));
        }
        luta[tid] = u32x2{hw[0], hw[1]};
        lutb[tid] = u32x2{lw[0], lw[1]};
    }

    // X operands of this wave: row blocks RB0 + rb, per k-block both planes
    const uint32_t nkb = a.in_pad / 16;
    const uint32_t RB0 = (r0 + wr) >> 5;
    const half8 *xrow[2];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const bool ok = r0 + wr + 32 * rb < a.rows;
        xrow[rb] = reinterpret_cast<const half8 *>(a.xs) + (uint64_t)(ok ? RB0 + rb : 0) * nkb * 128 + lane;
    }
    // this lane's two output columns, o0 + wo + 32 ob + ln: 32 codes per step
    // each (two words); lane half jh uses the 16-bit half jh of word ks
    const uint8_t *crow[OB];
    const uint16_t *nrow[OB];
#pragma unroll
    for (int ob = 0; ob < OB; ob++) {
        const uint32_t o = o0 + wo + 32 * ob + ln, oc = o < out ? o : 0;
        crow[ob] = a.packed[ti] + (uint64_t)oc * a.rowbytes;
        nrow[ob] = a.norms[ti] + (uint64_t)oc * a.ngroup;
    }
    struct Step {
        half8 x[2][2][2];               // [ks][rb][plane]
        uint2 c[OB];                    // [ob] codes
        uint16_t nb[OB];                // [ob] the norm of the step's group
    };
    auto load = [&](uint32_t k0, Step &st) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int p = 0; p < 2; p++)
                    st.x[ks][rb][p] = xrow[rb][((k0 >> 4) + ks) * 128 + 64 * p];
#pragma unroll
        for (int ob = 0; ob < OB; ob++) {
            st.c[ob] = *reinterpret_cast<const uint2 *>(crow[ob] + k0 / 4);
            st.nb[ob] = nrow[ob][k0 >> a.log2_group];
        }
    };

    float16v acc[2][OB], ysum[2][OB];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int ob = 0; ob < OB; ob++)
            ysum[rb][ob] = float16v{};
    // One step: 24 MFMAs; `first` starts the group's sums from zero (a literal
    // at each call site, so each variant carries no branch).
    auto compute = [&](const Step &st, const bool first) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            half8 wa[OB], wb[OB];
#pragma unroll
            for (int ob = 0; ob < OB; ob++) {
                const uint32_t c16 = ((ks ? st.c[ob].y : st.c[ob].x) >> (16 * jh)) & 0xFFFFu;
                // separate index registers for the two tables: merged into
                // one read per byte, the a and b parts would land in the
                // wrong registers and need moves into operand order
                uint32_t i0 = c16 & 0xFFu, i1 = c16 >> 8, j0 = i0, j1 = i1;
                asm volatile("" : "+v"(j0), "+v"(j1));
                const u32x2 a0 = luta[i0], a1 = luta[i1];
                const u32x2 b0 = lutb[j0], b1 = lutb[j1];
                wa[ob] = __builtin_bit_cast(half8, u32x4{a0.x, a0.y, a1.x, a1.y});
                wb[ob] = __builtin_bit_cast(half8, u32x4{b0.x, b0.y, b1.x, b1.y});
            }
            // the three products of each block in turn over the four blocks,
            // so consecutive MFMAs never wait on each other's results
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int ob = 0; ob < OB; ob++)
                    acc[rb][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        st.x[ks][rb][0], wa[ob], (first && ks == 0) ? float16v{} : acc[rb][ob], 0, 0, 0);
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int ob = 0; ob < OB; ob++)
                    acc[rb][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(st.x[ks][rb][1], wa[ob], acc[rb][ob], 0, 0, 0);
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int ob = 0; ob < OB; ob++)
                    acc[rb][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(st.x[ks][rb][0], wb[ob], acc[rb][ob], 0, 0, 0);
        }
    };
    // A group's end folds its sums into the totals with its norms, which
    // every step of the group loads beside its operands (so their wait is
    // that of the step's own data).
    auto fold = [&](const Step &st) {
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int ob = 0; ob < OB; ob++) {
                const float nrm = half_bits_to_float(st.nb[ob]);
#pragma unroll
                for (int i = 0; i < 16; i++)
                    ysum[rb][ob][i] = fmaf(nrm, acc[rb][ob][i], ysum[rb][ob][i]);
            }
    };
    const uint32_t nsteps = a.in_pad / CS_KT, gmask = (a.group / CS_KT) - 1;   // steps per group: a power of two
    auto step = [&](const Step &st, uint32_t s) __attribute__((always_inline)) {
        if ((s & gmask) == 0)
            compute(st, true);
        else
            compute(st, false);
        if (((s + 1) & gmask) == 0)
            fold(st);
    };

    // Steps in pairs, so the two register sets alternate without copies.
    // Every load is unconditional (a pair's last one re-reads a valid step
    // when nothing is left), so each wait covers exactly the step it feeds
    // and the next step's loads stay in flight. in_pad is a multiple of the
    // group, itself a multiple of one step.
    Step s0, s1;
    load(0, s0);
    __syncthreads();                    // the tables are written
    uint32_t s = 0;
    for (; s + 2 <= nsteps; s += 2) {
        load((s + 1) * CS_KT, s1);
        step(s0, s);
        load(min(s + 2, nsteps - 1) * CS_KT, s0);
        step(s1, s + 1);
    }
    if (s < nsteps)
        step(s0, s);
    // D layout: lane holds output column ln of each block, rows 8 (i/4) + 4 jh + (i%4)
#pragma unroll
    for (int ob = 0; ob < OB; ob++) {
        const uint32_t o = o0 + wo + 32 * ob + ln;
        if (o >= out)
            continue;
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t row = r0 + wr + 32 * rb + 8 * (i >> 2) + 4 * jh + (i & 3);
                if (row < a.rows)
                    y[(uint64_t)row * out + o] = ldexpf(ysum[rb][ob][i], -(a.rexp[row] + ecb));
            }
    }
}

hipError_t launch_cq_prepare_split(const CqPrepSplitArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    if (a.in_pad <= (uint32_t)CQ_REG_COLS && a.group >= 64) {
        hipLaunchKernelGGL(cq_prepare_split_reg_kernel, dim3((a.rows + 7) / 8), dim3(512), 0, s, a);
        return hipGetLastError();
    }
    CqPrepSplitArgs b = a;
    b.rpw = std::max(1u, std::min(4u, 16384u / a.in_pad));
    hipLaunchKernelGGL(cq_prepare_split_kernel, dim3((a.rows + b.rpw - 1) / b.rpw), dim3(256),
                       b.rpw * a.in_pad * sizeof(float), s, b);
    return hipGetLastError();
}

hipError_t launch_cq_gemm_split(const CqSplitArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.nt == 0 || a.tile0[a.nt] == 0)
        return hipSuccess;
    const uint64_t items = (uint64_t)((a.rows + CQ_SPLIT_MT - 1) / CQ_SPLIT_MT) * a.tile0[a.nt];
    const uint64_t grid = (items + 7) / 8 * 8;
    if (grid > 0x7FFFFFFFull)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(cq_gemm_split_kernel<CQ_SPLIT_OB>, dim3((uint32_t)grid), dim3(256), 0, s, a);
    return hipGetLastError();
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
