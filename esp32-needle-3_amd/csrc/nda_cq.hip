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
//   cq_lut2_kernel      the same for 2-bit tensors and a few rows, summed in
//                       the engine's own order (bit-identical y)
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
//   xh * 2^rexp[r]             = xa + xb   per row, from the split prepare
//   cb[c] * norm * 2^cexp[o]   = wa + wb   per (column, group), at tensor creation
//   sum_k w x  ~  sum_k (wa xa + wa xb + wb xa)   (wb xb, 2^-22 relative, dropped)
// Products and sums are fp32 inside the MFMA, and the total is scaled by
// 2^-(rexp + cexp) at the end. The powers of two put each row's and each
// column's largest |value| in [2^14, 2^15), so the large parts are normal
// fp16 numbers with their full 11 bits: the pairs hold 22 significant bits
// of the engine's fp32 values, and the result stays within fp32
// reassociation of the engine's matvec (a few 2^-22 of sum |w x|; the
// engine applies the norm to the group's dot product, here it sits in the
// weights).
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
// one wave per row, lane l holding columns 512 h + 8 l .. +7 (h < NH). The
// butterfly stages are the engine's (the same pairs, a + b and a - b, stage
// by stage): len < 8 inside a lane, 8 <= len < 512 between lanes l and
// l ^ (len / 8) (the upper lane's a - b as fmaf(-1, b, a), one rounding of
// the same exact difference), len >= 512 between a lane's column blocks.
// The values are the engine's bit for bit. A work-group is 8 consecutive
// rows (8 waves); their 16-byte operand slots meet in LDS, and each 128-byte
// line of the split rows (8 rows x one slot) is then written whole.
constexpr int CQ_REG_COLS = 1536;

template <int NH>       // column blocks of 512 in use: in_pad <= 512 NH
__global__ __launch_bounds__(512) void cq_prepare_split_reg_kernel(CqPrepSplitArgs a)
{
    // [plane][slot][row of 8 + pad], sized to the row: in_pad / 8 slots
    extern __shared__ __attribute__((aligned(16))) uint4 T[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.x * 8, row = row0 + wave;
    const bool live = row < a.rows;
    const float *x = a.x + (uint64_t)(live ? row : 0) * a.in;
    float v[NH][8];
    if ((a.in & 3) == 0) {
        // rows 16-byte aligned: 16-byte loads from clamped (in-bounds)
        // addresses, columns past the row's end selected to zero
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const uint32_t i0 = 512 * h + 8 * lane + 4 * f;
                const float4 p = *reinterpret_cast<const float4 *>(x + min(i0, a.in - 4));
                const bool ok = live && i0 + 4 <= a.in;
                v[h][4 * f + 0] = ok ? p.x : 0.0f;
                v[h][4 * f + 1] = ok ? p.y : 0.0f;
                v[h][4 * f + 2] = ok ? p.z : 0.0f;
                v[h][4 * f + 3] = ok ? p.w : 0.0f;
            }
    } else {
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const uint32_t i = 512 * h + 8 * lane + s;
                v[h][s] = live && i < a.in ? x[i] : 0.0f;
            }
    }
    // stage len = 2^lg, lg a compile-time index (so every register index is
    // fixed); group <= in_pad <= 1536 makes len <= 512
#pragma unroll
    for (int lg = 0; lg < 10; lg++) {
        const int len = 1 << lg;
        if ((uint32_t)len >= a.group)
            break;
        if (lg < 3) {
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int s = 0; s < 8; s++)
                    if ((s & len) == 0) {
                        const float u = v[h][s], w = v[h][s + len];
                        v[h][s] = u + w;
                        v[h][s + len] = u - w;
                    }
        } else if (lg < 9) {
            const int m = len >> 3;
            const float sg = (lane & m) ? -1.0f : 1.0f;
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    // lg is fixed in each unrolled stage: one cross-lane
                    // operation of distance m
                    float w;
                    switch (lg) {
                    case 3: w = xor_lanes<1>(v[h][s], lane); break;
                    case 4: w = xor_lanes<2>(v[h][s], lane); break;
                    case 5: w = xor_lanes<4>(v[h][s], lane); break;
                    case 6: w = xor_lanes<8>(v[h][s], lane); break;
                    case 7: w = xor_lanes<16>(v[h][s], lane); break;
                    default: w = xor_lanes<32>(v[h][s], lane); break;
                    }
                    v[h][s] = fmaf(sg, v[h][s], w);     // lower lane: v + w; upper: w - v
                }
        } else {
            if constexpr (NH >= 2) {
#pragma unroll
                for (int s = 0; s < 8; s++) {           // len 512: blocks 0 and 1
                    const float u = v[0][s], w = v[1][s];
                    v[0][s] = u + w;
                    v[1][s] = u - w;
                }
            }
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int h = 0; h < NH; h++)
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
    const uint32_t nslot = a.in_pad / 8;
#pragma unroll
    for (int h = 0; h < NH; h++) {
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
        T[c * 9 + wave] = __builtin_bit_cast(uint4, half8{h8[0], h8[1], h8[2], h8[3], h8[4], h8[5], h8[6], h8[7]});
        T[(nslot + c) * 9 + wave] = __builtin_bit_cast(uint4, half8{l8[0], l8[1], l8[2], l8[3], l8[4], l8[5], l8[6], l8[7]});
    }
    if (live && lane == 0)
        a.rexp[row] = sh;
    __syncthreads();
    // 8 rows' slot c of a plane is one 128-byte line (lanes row0 % 32 ..
    // +7 of one operand): thread t writes row t % 8 of line t / 8
    const uint32_t nkb = a.in_pad / 16;
    for (uint32_t u = threadIdx.x; u < 2 * nslot * 8; u += 512) {
        const uint32_t r = u & 7, c = (u >> 3) % nslot, p = (u >> 3) / nslot;
        *reinterpret_cast<uint4 *>(a.xs + split_index(row0 + r, 8 * c, nkb, (int)p)) = T[(p * nslot + c) * 9 + r];
    }
}

constexpr int CS_KT = 32;           // reduction columns per step: two MFMA k-blocks

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Decode data of a 2-bit tensor, written once when the tensor is created
// (one thread per output column o):
//   cexp[o]          power of two that puts the column's largest |cb[c] *
//                    norm| in [2^14, 2^15) (0 for an all-zero column)
//   tab[g][o]        the four weights cb[c] * norm[o][g] of group g (the
//                    engine's fp32 product, scaled by 2^cexp[o]), each as an
//                    fp16 pair a + b, laid out as two v_perm byte tables:
//                    {a high bytes, a low bytes, b high bytes, b low bytes},
//                    entry c at byte c of each
//   cw[s][o][h]      for step s (columns 32 s ..) and lane half h: the
//                    lane's 16 codes as one word, code b of group q (the
//                    columns 32 s + 16 (q / 2) + 8 h + 4 (q % 2) + b) at bit
//                    8 b + 2 q, so (w >> 2 q) & 0x03030303 puts four codes
//                    in four bytes; with them and the same bytes + 4, two
//                    v_perms give the selectors {c, c + 4, c', c' + 4} of
//                    two operand dwords (the low then the high byte of
//                    entry c, then those of entry c')
// so one v_perm per operand dword decodes two weights in either plane.
__global__ __launch_bounds__(256) void cq_split_tables_kernel(CqTabArgs a)
{
    const uint32_t o = blockIdx.x * 256 + threadIdx.x;
    if (o >= a.out)
        return;
    const float cb[4] = {a.cb[0], a.cb[1], a.cb[2], a.cb[3]};
    const uint16_t *nr = a.norms + (uint64_t)o * a.ngroup;
    float m = 0.0f;
    for (uint32_t g = 0; g < a.ngroup; g++) {
        const float nf = half_bits_to_float(nr[g]);
#pragma unroll
        for (int c = 0; c < 4; c++)
            m = fmaxf(m, fabsf(cb[c] * nf));
    }
    int e = 0, sh = 0;
    if (m > 0.0f && m <= FLT_MAX) {
        (void)frexpf(m, &e);
        sh = 15 - e;
    }
    a.cexp[o] = sh;
    for (uint32_t g = 0; g < a.ngroup; g++) {
        const float nf = half_bits_to_float(nr[g]);
        uint32_t t[4] = {0u, 0u, 0u, 0u};               // a hi, a lo, b hi, b lo bytes
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float v = ldexpf(cb[c] * nf, sh);
            asm volatile("" : "+v"(v));                 // both halves from this one value
            const _Float16 h = (_Float16)v, l = (_Float16)(v - (float)h);
            const uint32_t hb = __builtin_bit_cast(uint16_t, h), lb = __builtin_bit_cast(uint16_t, l);
            t[0] |= (hb >> 8) << (8 * c);
            t[1] |= (hb & 0xFFu) << (8 * c);
            t[2] |= (lb >> 8) << (8 * c);
            t[3] |= (lb & 0xFFu) << (8 * c);
        }
        a.tab[(uint64_t)g * a.out + o] = uint4{t[0], t[1], t[2], t[3]};
    }
    const uint8_t *row = a.packed + (uint64_t)o * a.rowbytes;
    const uint32_t nsteps = a.in_pad / CS_KT;
    for (uint32_t s = 0; s < nsteps; s++)
        for (uint32_t h = 0; h < 2; h++) {
            uint32_t w = 0;
            for (uint32_t q = 0; q < 4; q++)
                for (uint32_t b = 0; b < 4; b++) {
                    const uint32_t k = CS_KT * s + 16 * (q >> 1) + 8 * h + 4 * (q & 1) + b;
                    w |= ((row[k >> 2] >> (2 * (k & 3))) & 3u) << (8 * b + 2 * q);
                }
            a.cw[((uint64_t)s * a.out + o) * 2 + h] = w;
        }
}

// Work item = 128 rows x 128 outputs of one tensor, 4 waves of 64 x 64
// (2 x 2 blocks of 32 x 32), each wave independent of the others: it loads
// its X operands straight from the split rows and its weights' codes and
// group tables (one step ahead, in two register sets used in turn) and
// decodes each W operand dword with one v_perm (its selector from the
// codes by a shift, a mask and a v_perm per two dwords). The norms are inside the
// tables, so one sum per block runs over all groups. LDS holds only each
// wave's output stage (below); there is no barrier.
//
// Steps 2 apart use the same register set, and a group spans an even number
// of steps when it spans more than 2 (group / 32, with in_pad a multiple of
// the group). So a group's tables are loaded on its first two steps only,
// one per set, and each set keeps them for the group's later steps (half the
// table bytes at group 128). Likewise an item's row and column exponents are
// loaded on its first two steps and kept in both sets to its end. 6.5% off
// the q/k/v/gate launch at 49,787 rows.
//
// The grid is persistent: work-group w runs on XCD w % 8 and walks the
// items of that XCD's contiguous range, w / 8, w / 8 + G8, ... (G8
// work-groups per XCD). Consecutive items are the output tiles of one row
// tile, so the work-groups of an XCD running side by side read the same X
// rows from its L2. The prefetch runs across items: during an item's last
// step the next item's first step is loaded, and the exponents its stores
// need were loaded with its first two steps, so an item's end waits on no
// load. Loads for rows or outputs past the end read row or
// column 0 instead (in bounds); what they feed lands only in rows or
// columns that are never stored.
template <int OB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OB >= 2 ? 2 : 3)))
void cq_gemm_split_kernel(CqSplitArgs a)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31, jh = lane >> 5;
    const int wr = (wave & 1) * 64, wo = (wave >> 1) * 32 * OB;
    const uint32_t ntiles = a.tile0[a.nt];
    const uint32_t total = (a.rows + CQ_SPLIT_MT - 1) / CQ_SPLIT_MT * ntiles;
    const uint32_t G8 = gridDim.x / 8u, T8 = (total + 7u) / 8u, xcd = blockIdx.x % 8u;
    const uint32_t first = xcd * T8 + blockIdx.x / 8u, last = min(total, (xcd + 1u) * T8);
    if (first >= last)
        return;
    const uint32_t nkb = a.in_pad / 16, nsteps = a.in_pad / CS_KT;
    const uint32_t gmask = ((1u << a.log2_group) / CS_KT) - 1u;   // steps of a group - 1 (group >= 32)

    // item it: row tile it / ntiles, output tile it % ntiles (tensor ti)
    struct Item {
        uint32_t r0, o0, ti, out;
    };
    auto item = [&](uint32_t it) {
        Item m;
        const uint32_t rt = it / ntiles, ot = it % ntiles;
        uint32_t ti = 0;
        while (ti + 1 < a.nt && ot >= a.tile0[ti + 1])
            ti++;
        m.r0 = rt * CQ_SPLIT_MT;
        m.ti = ti;
        m.out = a.out[ti];
        m.o0 = (ot - a.tile0[ti]) * (64 * OB);
        return m;
    };
    // where an item's operands are: this wave's X row blocks, and this
    // lane's output columns m.o0 + wo + 32 ob + ln (byte offsets of their
    // selectors, lane half jh, and group tables)
    struct Src {
        const half8 *xr[2];
        const char *cb, *tb;
        const int32_t *ce;
        uint64_t ss, ts;
        uint32_t soff[OB], toff[OB], oc[OB], row;
    };
    auto source = [&](const Item &m) {
        Src q;
        const uint32_t RB0 = (m.r0 + wr) >> 5;
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const bool ok = m.r0 + wr + 32 * rb < a.rows;
            q.xr[rb] = reinterpret_cast<const half8 *>(a.xs) + (uint64_t)(ok ? RB0 + rb : 0) * nkb * 128;
        }
        q.cb = reinterpret_cast<const char *>(a.cw[m.ti]);
        q.tb = reinterpret_cast<const char *>(a.tab[m.ti]);
        q.ce = a.cexp[m.ti];
        q.ss = (uint64_t)m.out * 8;
        q.ts = (uint64_t)m.out * 16;
#pragma unroll
        for (int ob = 0; ob < OB; ob++) {
            const uint32_t o = m.o0 + wo + 32 * ob + ln, oc = o < m.out ? o : 0;
            q.oc[ob] = oc;
            q.soff[ob] = (oc * 2 + jh) * 4;
            q.toff[ob] = oc * 16;
        }
        q.row = min(m.r0 + wr + lane, a.rows - 1);      // lane t: row r0 + wr + t
        return q;
    };
    struct Step {
        half8 x[2][2][2];               // [ks][rb][plane]
        uint32_t cw[OB];                // [ob] the step's 16 codes
        uint4 tab[OB];
        int32_t rx, ce[OB];             // the item's row and column exponents
    };
    auto load = [&](const Src &q, uint32_t s, Step &st) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int p = 0; p < 2; p++)
                    st.x[ks][rb][p] = q.xr[rb][((2 * s + ks) * 2 + p) * 64 + lane];
        const char *cb = q.cb + s * q.ss;
#pragma unroll
        for (int ob = 0; ob < OB; ob++)
            st.cw[ob] = *reinterpret_cast<const uint32_t *>(cb + q.soff[ob]);
        if ((s & gmask) < 2) {          // the group's first two steps (above)
            const char *tb = q.tb + ((s * CS_KT) >> a.log2_group) * q.ts;
#pragma unroll
            for (int ob = 0; ob < OB; ob++)
                st.tab[ob] = *reinterpret_cast<const uint4 *>(tb + q.toff[ob]);
        }
        if (s < 2) {                    // the item's first two steps
#pragma unroll
            for (int ob = 0; ob < OB; ob++)
                st.ce[ob] = q.ce[q.oc[ob]];
            st.rx = a.rexp[q.row];
        }
    };

    float16v acc[2][OB];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int ob = 0; ob < OB; ob++)
            acc[rb][ob] = float16v{};
    // One step: 24 MFMAs (OB = 2), the three products of each block in
    // turn over the four blocks, so consecutive MFMAs never wait on each
    // other's results.
    auto compute = [&](const Step &st) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            half8 wa[OB], wb[OB];
#pragma unroll
            for (int ob = 0; ob < OB; ob++) {
                const uint4 tb = st.tab[ob];
                const uint32_t b0 = (st.cw[ob] >> (4 * ks)) & 0x03030303u, h0 = b0 | 0x04040404u;
                const uint32_t b1 = (st.cw[ob] >> (4 * ks + 2)) & 0x03030303u, h1 = b1 | 0x04040404u;
                const uint4 sl = {__builtin_amdgcn_perm(h0, b0, 0x05010400u), __builtin_amdgcn_perm(h0, b0, 0x07030602u),
                                  __builtin_amdgcn_perm(h1, b1, 0x05010400u), __builtin_amdgcn_perm(h1, b1, 0x07030602u)};
                const u32x4 ua = {__builtin_amdgcn_perm(tb.x, tb.y, sl.x), __builtin_amdgcn_perm(tb.x, tb.y, sl.y),
                                  __builtin_amdgcn_perm(tb.x, tb.y, sl.z), __builtin_amdgcn_perm(tb.x, tb.y, sl.w)};
                const u32x4 ub = {__builtin_amdgcn_perm(tb.z, tb.w, sl.x), __builtin_amdgcn_perm(tb.z, tb.w, sl.y),
                                  __builtin_amdgcn_perm(tb.z, tb.w, sl.z), __builtin_amdgcn_perm(tb.z, tb.w, sl.w)};
                wa[ob] = __builtin_bit_cast(half8, ua);
                wb[ob] = __builtin_bit_cast(half8, ub);
            }
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int ob = 0; ob < OB; ob++)
                    acc[rb][ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(st.x[ks][rb][0], wa[ob], acc[rb][ob], 0, 0, 0);
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
    // An item's end: the sums, scaled by 2^-(rexp + cexp), go to this
    // wave's LDS stage as [64 rows][32 OB columns] and acc is zeroed. The
    // stage goes out during the next item's first steps, two 16-byte
    // streaming stores (8 / OB rows of 32 OB columns each) at a step: a
    // quarter of the store instructions of storing from the MFMA layout,
    // spread between the MFMA runs, and the output stream does not displace
    // the X rows the XCD's work-groups re-read from L2. A wave reads back
    // only its own stage, and its LDS operations complete in order.
    constexpr int SLD = 32 * OB + 4;            // row stride of the stage, floats
    constexpr int NG = 4 * OB;                  // groups of two stores per item
    __shared__ float stage[4 * 64 * SLD];
    float *const sw = stage + wave * 64 * SLD;
    Item mo = {0, 0, 0, 0};
    uint32_t pend = 0;
    auto drain = [&]() __attribute__((always_inline)) {
        const uint32_t g = NG - pend;
        float *y = a.y[mo.ti];
        const bool v4 = (mo.out & 3u) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t r = (2 * g + h) * (8 / OB) + lane / (8 * OB), c = 4 * (lane % (8 * OB));
            const float4v v = *reinterpret_cast<const float4v *>(sw + r * SLD + c);
            const uint32_t row = mo.r0 + wr + r, o = mo.o0 + wo + c;
            if (row < a.rows) {
                float *dst = y + (uint64_t)row * mo.out + o;
                if (v4 && o + 3 < mo.out) {
                    __builtin_nontemporal_store(v, reinterpret_cast<float4v *>(dst));
                } else {
                    if (o < mo.out)
                        __builtin_nontemporal_store(v.x, dst + 0);
                    if (o + 1 < mo.out)
                        __builtin_nontemporal_store(v.y, dst + 1);
                    if (o + 2 < mo.out)
                        __builtin_nontemporal_store(v.z, dst + 2);
                    if (o + 3 < mo.out)
                        __builtin_nontemporal_store(v.w, dst + 3);
                }
            }
        }
        pend--;
    };
    auto finish = [&](const Item &m, const Step &st) {
        while (pend)
            drain();
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int t = 32 * rb + 8 * (i >> 2) + 4 * jh + (i & 3);
                const int rx = __shfl(st.rx, t, 64);
#pragma unroll
                for (int ob = 0; ob < OB; ob++)
                    sw[t * SLD + 32 * ob + ln] = ldexpf(acc[rb][ob][i], -(rx + st.ce[ob]));
            }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int ob = 0; ob < OB; ob++)
                acc[rb][ob] = float16v{};
        mo = m;
        pend = NG;
    };

    // Loads run one step ahead of the MFMAs at (lit, ls); when nothing is
    // left they re-read the last step, so every load is unconditional and
    // each wait covers exactly the step it feeds. The scheduling barriers
    // keep each step's loads ahead of the previous step's MFMAs (left to
    // itself the scheduler sinks them next to their use).
    uint32_t lit = first, ls = 0, cit = first, cs = 0;
    Item mc = item(first);
    Src q = source(mc);
    auto next_load = [&]() {
        if (++ls == nsteps) {
            if (lit + G8 < last) {
                lit += G8;
                ls = 0;
                q = source(item(lit));
            } else {
                ls = nsteps - 1;
            }
        }
    };
    Step s0, s1;
    load(q, ls, s0);
    next_load();
    for (;;) {
        load(q, ls, s1);
        next_load();
        __builtin_amdgcn_sched_barrier(0);
        compute(s0);
        __builtin_amdgcn_sched_barrier(0);
        if (pend)
            drain();
        if (++cs == nsteps) {
            finish(mc, s0);
            if (cit + G8 >= last)
                break;
            cit += G8;
            cs = 0;
            mc = item(cit);
        }
        load(q, ls, s0);
        next_load();
        __builtin_amdgcn_sched_barrier(0);
        compute(s1);
        __builtin_amdgcn_sched_barrier(0);
        if (pend)
            drain();
        if (++cs == nsteps) {
            finish(mc, s1);
            if (cit + G8 >= last)
                break;
            cit += G8;
            cs = 0;
            mc = item(cit);
        }
    }
    while (pend)
        drain();
}

// ------------------------------------------------ the engine's LUT order

// 2-bit matvecs for a few rows (one decode step's tokens) computed the way
// the engine computes them (nd_cq_lut_build + nd_lut2_rows_c, engine/src/
// nd_quant.c:75-94, :722-764), so y is bit-identical to the engine's: per
// row the pair table T[p][i0 + 4 i1] = cb[i0] xh[2p] + cb[i1] xh[2p+1] in
// LDS; per output the groups in order, each group's 32-bit words in order,
// nibble k of a word added into accumulator k % 4 from table block k, and
// acc = acc + norm * ((s0 + s1) + (s2 + s3)). One work-group per
// (256-output tile, row), one output per thread; every product and sum
// rounds on its own.
__global__ __launch_bounds__(256) void cq_lut2_kernel(CqGemmArgs a)
{
#pragma clang fp contract(off)
    extern __shared__ float lut[];   // [in_pad / 2][16]
    const uint32_t tile = blockIdx.x, row = blockIdx.y;
    uint32_t t = 0;
    while (t + 1 < a.nt && tile >= a.tile0[t + 1])
        t++;
    const float *xh = a.xh + (uint64_t)row * a.in_pad;
    const float *cb = a.cb[t];
    for (uint32_t e = threadIdx.x; e < a.in_pad * 8; e += 256) {
        const uint32_t p = e >> 4;
        const float x0 = xh[2 * p], x1 = xh[2 * p + 1];
        const float lo = cb[e & 3] * x0, hi = cb[(e >> 2) & 3] * x1;
        lut[e] = lo + hi;
    }
    __syncthreads();
    const uint32_t o = (tile - a.tile0[t]) * CQ_LUT_OT + threadIdx.x;
    if (o >= a.out[t])
        return;
    const uint32_t *q = reinterpret_cast<const uint32_t *>(a.packed[t] + (uint64_t)o * a.rowbytes);
    const uint16_t *nrm = a.norms[t] + (uint64_t)o * a.ngroup;
    const uint32_t gw = a.group / 16;          // words per group
    const float *T = lut;
    float acc = 0.0f;
    for (uint32_t gi = 0; gi < a.ngroup; gi++) {
        const float nf = half_bits_to_float(nrm[gi]);
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        for (uint32_t j = 0; j < gw; j++) {
            const uint32_t w = q[j];
            s0 = s0 + T[w & 15u];
            s1 = s1 + T[16 + ((w >> 4) & 15u)];
            s2 = s2 + T[32 + ((w >> 8) & 15u)];
            s3 = s3 + T[48 + ((w >> 12) & 15u)];
            T += 64;
            s0 = s0 + T[(w >> 16) & 15u];
            s1 = s1 + T[16 + ((w >> 20) & 15u)];
            s2 = s2 + T[32 + ((w >> 24) & 15u)];
            s3 = s3 + T[48 + (w >> 28)];
            T += 64;
        }
        q += gw;
        acc = acc + nf * ((s0 + s1) + (s2 + s3));
    }
    a.y[t][(uint64_t)row * a.out[t] + o] = acc;
}

hipError_t launch_cq_lut2(const CqGemmArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.nt == 0 || a.tile0[a.nt] == 0)
        return hipSuccess;
    if (a.bits != 2 || a.group % 16 || a.in_pad > CQ_LUT_MAX_IN || a.rows > 65535)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(cq_lut2_kernel, dim3(a.tile0[a.nt], a.rows), dim3(256), (size_t)a.in_pad * 8 * sizeof(float),
                       s, a);
    return hipGetLastError();
}

hipError_t launch_cq_split_tables(const CqTabArgs &a, hipStream_t s)
{
    if (a.out == 0)
        return hipSuccess;
    hipLaunchKernelGGL(cq_split_tables_kernel, dim3((a.out + 255) / 256), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_cq_prepare_split(const CqPrepSplitArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    if (a.in_pad <= (uint32_t)CQ_REG_COLS && a.group >= 64) {
        const size_t lds = (size_t)a.in_pad / 8 * 2 * 9 * sizeof(uint4);
        const dim3 grid((a.rows + 7) / 8);
        if (a.in_pad <= 512)
            hipLaunchKernelGGL(cq_prepare_split_reg_kernel<1>, grid, dim3(512), lds, s, a);
        else if (a.in_pad <= 1024)
            hipLaunchKernelGGL(cq_prepare_split_reg_kernel<2>, grid, dim3(512), lds, s, a);
        else
            hipLaunchKernelGGL(cq_prepare_split_reg_kernel<3>, grid, dim3(512), lds, s, a);
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
    if (items > 0x7FFFFFFFull)
        return hipErrorInvalidValue;
    // persistent: at most two work-groups per CU (the kernel's occupancy),
    // a multiple of 8 so that every XCD holds the same number
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return hipErrorInvalidDevice;
    if (cus[dev] <= 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return hipErrorInvalidDevice;
    const uint64_t slots = std::max<uint64_t>(8, (uint64_t)cus[dev] * 2 / 8 * 8);
    const uint64_t grid = std::min<uint64_t>((items + 7) / 8 * 8, slots);
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
