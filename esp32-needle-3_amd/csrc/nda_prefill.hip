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
// Key tiles of 32 slots of one segment (shared prefix, then own) are staged
// through LDS (K and V row-major; V is read transposed), then per wave and
// tile:
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

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

// four fp16 of a transposed 16-lane block (ds_read_b64_tr_b16): see the P.V
// operand of the prefill kernel for the lane layout
__device__ __forceinline__ half4 tr16_read(const _Float16 *p)
{
    const short4v w = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4v *)(__attribute__((address_space(3))) void *)p);
    return __builtin_bit_cast(half4, w);
}

// s_waitcnt vmcnt(0), the other counters unconstrained (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8), fenced so that
// neither the optimiser nor the scheduler moves memory accesses across it
__device__ __forceinline__ void wait_vmcnt0()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(lds_void *)p;
}

// A direct-to-LDS load: lane l's 16 bytes at base + voff land at LDS byte
// m0 + 16 l. Issued from inline asm, which the compiler's wait insertion
// does not follow into LDS: without alias information it would wait for
// every such load in flight before any LDS read. The caller waits for
// completion (wait_vmcnt0); waits the compiler places for its own loads stay
// correct, since extra loads in the in-order count only make them stricter.
// m0 is written by a scalar instruction one wait state ahead of the load
// (nothing else in this kernel uses m0).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const uint8_t *base, uint32_t voff, uint32_t m0)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(m0)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ float16v mfma32(half8 a, half8 b, float16v c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));

typedef const __attribute__((address_space(4))) int32_t *cptr;   // read through scalar loads

// int8 codes as fp16, exact: 0x64 over the byte code ^ 0x80 is the fp16
// 1024 + code + 128, so one xor, a byte permute and a packed fp16 subtract
// per two codes.
template <int SEL>
__device__ __forceinline__ half2v codes2(uint32_t xs)   // xs = codes ^ 0x80808080
{
    const uint32_t u = __builtin_amdgcn_perm(0x64646464u, xs, (uint32_t)SEL);
    return __builtin_bit_cast(half2v, u) - half2v{(_Float16)1152.0f, (_Float16)1152.0f};
}

// eight int8 codes (bytes 0..7 of w) as fp16, in byte order
__device__ __forceinline__ half8 codes8(u32x2 w)
{
    const uint32_t x0 = w.x ^ 0x80808080u, x1 = w.y ^ 0x80808080u;
    const half2v c0 = codes2<0x04010400>(x0), c1 = codes2<0x04030402>(x0);
    const half2v c2 = codes2<0x04010400>(x1), c3 = codes2<0x04030402>(x1);
    return half8{c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>)
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// Key tiles are 32 slots of one segment -- the shared prefix's slots, then
// the sequence's own (own slot s holds position n_sh + s) -- aligned to 32
// within it. A half tile (16 keys) is then 16 consecutive slots of one page,
// and its K rows, V rows and (int8) k and v scales are contiguous runs of
// that page's kv-head block. A thread's share of a tile is a few 16-byte
// chunks of those runs at offsets fixed for the launch, from one base per
// half tile that one scalar page-table read gives.
// DMA: fp16 rows of 64 halves go from global memory straight into LDS
// (global_load_lds_dwordx4), with no staging registers, for 2- and 4-wave
// groups with a tile table, which then fit 4 waves per SIMD instead of 3 (a
// shared-prefix prefill of 48-token suffixes: 0.112-0.114 against
// 0.118-0.119 ms). One buffer is then K [32][64] and V [32][64] halves,
// unpadded, a row's 16-byte chunk c at chunk position c ^ (row % 8) (see
// PfIO::load_lds). The 8-wave groups, at 4 waves per SIMD either way, keep
// their one staged chunk per thread: direct loads made the 512-token chunk
// 3% slower (563-566 against 581-585 TFLOP/s). Without a table the page ids'
// ring spills at 128 registers, so those groups stay staged too.
template <int ES, int DK, int DV, int NTHR, bool TAB>
constexpr bool pf_direct = ES == 2 && DK == 64 && DV == 64 && NTHR < 512 && TAB;

template <int ES, int DK, int DV, int NTHR, bool DIRECT = false>
struct PfTile {
    static constexpr int KPAD = DK + 8;        // halves per K row in LDS
    static constexpr int VPAD = DV + 8;        // halves per V row in LDS (row-major; read transposed)
    static constexpr int KC = DK * ES / 16;    // 16-byte chunks per stored K row
    static constexpr int VC = DV * ES / 16;
    static constexpr int HCH = 16 * (KC + VC) + (ES == 1 ? 8 : 0);   // chunks of a half tile
    static constexpr int HP = (HCH + 63) / 64 * 64;   // padded to whole waves: a wave's chunks share a half
    static constexpr int CPT = (2 * HP + NTHR - 1) / NTHR;             // chunks per thread
    static constexpr bool DMA = DIRECT;   // see pf_direct
    // one LDS buffer otherwise: K [32][KPAD] halves, V [32][VPAD] halves,
    // k scales, v scales
    static constexpr int VOFF = DMA ? PF_KT * 128 : PF_KT * KPAD * 2, SOFF = VOFF + PF_KT * VPAD * 2;
    static constexpr int BUF = DMA ? 2 * PF_KT * 128 : SOFF + 2 * PF_KT * 4;
    static_assert(DK * ES % 16 == 0 && DV * ES % 16 == 0, "rows are whole 16-byte chunks");
    static_assert(NTHR % 64 == 0 && BUF % 16 == 0, "");
};

// One thread's share of a K/V tile in flight: raw 16-byte chunks, and the
// tile's count of slots before its segment's end (uniform).
template <int CPT>
struct Staged {
    u32x4 w[CPT];
    int vlim;
};

// Chunk c of a tile (c = tid + i * NTHR): where it is read from, relative to
// its half tile's kv-head block at in-page slot 0, and where it goes in LDS.
// Padding chunks (and chunks past the tile) read chunk 0 and store nothing.
struct PfChunk {
    int half;           // uniform per wave
    uint32_t gofs, rb;  // byte offset, plus rb bytes per in-page slot of the half
    int lds;            // byte offset in an LDS buffer; -1: not stored
    int key;            // the chunk's (first) key in the tile
    bool scale;         // four fp32 scales rather than codes
};

template <int ES, int DK, int DV, int NTHR, int I>
__device__ __forceinline__ PfChunk pf_chunk(int tid, int wave, uint32_t P)
{
    using T = PfTile<ES, DK, DV, NTHR>;
    PfChunk k;
    const int c = tid + I * NTHR;
    const int cc = c < 2 * T::HP ? c : 2 * T::HP - 1;
    // the half is known at compile time when chunks [I NTHR, (I+1) NTHR)
    // lie in one half; else it follows from the (uniform) wave index
    constexpr int C0 = I * NTHR, C1 = (I + 1) * NTHR - 1;
    constexpr int H0 = (C0 < 2 * T::HP ? C0 : 2 * T::HP - 1) / T::HP;
    constexpr int H1 = (C1 < 2 * T::HP ? C1 : 2 * T::HP - 1) / T::HP;
    if constexpr (H0 == H1) {
        k.half = H0;
    } else {
        const int cw = 64 * wave + I * NTHR;
        k.half = (cw < 2 * T::HP ? cw : 2 * T::HP - 1) / T::HP;
    }
    int q = cc % T::HP;
    const bool pad = c >= 2 * T::HP || q >= T::HCH;
    if (pad)
        q = 0;
    k.scale = false;
    if (q < 16 * T::KC) {
        const int row = q / T::KC, col = q % T::KC;
        k.gofs = 16u * q;
        k.rb = DK * ES;
        k.key = 16 * k.half + row;
        k.lds = k.key * T::KPAD * 2 + col * 16 * (3 - ES);
    } else if (q < 16 * (T::KC + T::VC)) {
        const int q2 = q - 16 * T::KC, row = q2 / T::VC, col = q2 % T::VC;
        k.gofs = P * (DK * ES) + 16u * q2;
        k.rb = DV * ES;
        k.key = 16 * k.half + row;
        k.lds = T::VOFF + k.key * T::VPAD * 2 + col * 16 * (3 - ES);
    } else {
        const int s = q - 16 * (T::KC + T::VC);   // 0-3: k scales, 4-7: v scales (int8 only)
        k.gofs = P * (DK + DV) + (s >= 4 ? 4u * P : 0u) + 16u * (s & 3);
        k.rb = 4;
        k.key = 16 * k.half + 4 * (s & 3);
        k.lds = T::SOFF + (s >= 4 ? 4 * PF_KT : 0) + 4 * k.key;
        k.scale = true;
    }
    if (pad)
        k.lds = -1;
    return k;
}

template <int ES, int DK, int DV, int NTHR, bool TAB>
struct PfIO {
    using T = PfTile<ES, DK, DV, NTHR, pf_direct<ES, DK, DV, NTHR, TAB>>;
    // A tile's page ids and first in-page slots (uniform), as read a tile
    // before its data is requested: the ids are used only then, so their
    // reads have a tile to land. They are vector loads (of one address):
    // the in-order vector-memory counter lets a later wait skip them, where
    // a scalar read would be waited for by the next LDS wait (scalar reads
    // return out of order, so that wait must drain them all). Their address
    // carries threadIdx.y (zero in these one-dimensional launches), so the
    // compiler keeps the ids in vector registers and moves them to scalar
    // ones only where load() reads them, instead of right after the read
    // (which would wait for it there). Half 1's slot is a difference from
    // half 0's. Choices between two fields are made as base + (c ?
    // difference : 0) throughout: a select between two loaded fields is
    // folded into one load through a selected field address, which leaves
    // the whole object in scratch memory.
    struct TileRef {
        uint32_t p0, p1;
        uint32_t sip0, dsip;
        int vlim;               // slots before the segment's end, from the tile's first
    };
    const uint8_t *pool;
    const int32_t *own_pages;
    int64_t pre_minus_own;      // prefix page-table row - own row, in entries
    uint32_t zero;              // threadIdx.y: 0
    uint64_t head_off;
    uint32_t page_bytes, log2_page;
    int tid, wave, n_sh, own_len;
    // processing order: full shared tiles [0, nfs), own tiles visible to
    // every row [nfs, jfull), then the masked ones: the partial shared tile
    // (psh = 1 if there is one), then the own tiles crossing the diagonal
    int nfs, psh, jfull, ntile;

    // tile t of the processing order: segment, first slot, segment length
    // (selects, no branches: this runs on the scalar unit every tile)
    __device__ __forceinline__ void seg(int t, bool &sh, int &s0, int &len) const
    {
        const bool tail = psh != 0 && t == jfull;       // the partial shared tile
        sh = t < nfs || tail;
        const int own = t - nfs - (t > jfull ? psh : 0);
        s0 = PF_KT * (sh ? (tail ? nfs : t) : own);
        len = own_len + (sh ? n_sh - own_len : 0);
    }
    // TAB: every tile's TileRef, built once per work-group in LDS, entries
    // [0, tab_n); fetch() is then one broadcast LDS read instead of the
    // segment arithmetic and two page-table loads per tile
    const uint4 *tab;
    int tab_n;
    __device__ __forceinline__ void fetch(int t, TileRef &r) const
    {
        if constexpr (TAB) {
            const uint4 e = tab[min(t, tab_n - 1)];
            r.p0 = e.x;
            r.p1 = e.y;
            r.sip0 = e.z & 0xFFFFu;
            r.dsip = e.z >> 16;
            r.vlim = (int)e.w;
        } else {
            compute(t, r);
        }
    }
    // a table entry (as read from LDS) as uniform values
    __device__ __forceinline__ static TileRef uniform(const uint4 &e)
    {
        TileRef r;
        r.p0 = __builtin_amdgcn_readfirstlane(e.x);
        r.p1 = __builtin_amdgcn_readfirstlane(e.y);
        const uint32_t z = __builtin_amdgcn_readfirstlane(e.z);
        r.sip0 = z & 0xFFFFu;
        r.dsip = z >> 16;
        r.vlim = (int)__builtin_amdgcn_readfirstlane(e.w);
        return r;
    }
    // page ids of tile t (past the last tile: the last tile again); a half
    // past its segment's end rereads half 0
    __device__ __forceinline__ void compute(int t, TileRef &r) const
    {
        bool sh;
        int s0, len;
        seg(min(t, ntile - 1), sh, s0, len);
        const int s1 = s0 + 16 < len ? s0 + 16 : s0;
        const int32_t *rows = own_pages + (sh ? pre_minus_own : 0);
        r.p0 = (uint32_t)rows[((uint32_t)s0 >> log2_page) + zero];
        r.p1 = (uint32_t)rows[((uint32_t)s1 >> log2_page) + zero];
        const uint32_t m = (1u << log2_page) - 1;
        r.sip0 = (uint32_t)s0 & m;
        r.dsip = ((uint32_t)s1 & m) - r.sip0;
        r.vlim = len - s0;
    }
    // Plain loads, not nontemporal ones: a tile is read again by other
    // work-groups (every sequence reads the shared prefix's tiles; the row
    // groups of one sequence and kv-head read the same own tiles), and L2
    // keeps it for them. With the nontemporal hint a shared-prefix prefill
    // of 48-token suffixes took 0.142 ms instead of 0.122, and a 512-token
    // chunk 3-4% longer.
    __device__ __forceinline__ void load(const TileRef &r, Staged<T::CPT> &sg) const
    {
        const uint32_t P = 1u << log2_page;
        // a page is under 4 GiB: one 32 x 32 -> 64-bit multiply-add
        const uint32_t p0 = __builtin_amdgcn_readfirstlane(r.p0), p1 = __builtin_amdgcn_readfirstlane(r.p1);
        const uint8_t *hb0 = pool + ((uint64_t)p0 * page_bytes + head_off);
        const int64_t dhb = ((int64_t)p1 - (int64_t)p0) * (int64_t)page_bytes;
        static_for<T::CPT>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            const PfChunk k = pf_chunk<ES, DK, DV, NTHR, i>(tid, wave, P);
            const uint8_t *hb = hb0 + (k.half ? dhb : 0);
            const uint32_t off = k.gofs + (r.sip0 + (k.half ? r.dsip : 0u)) * k.rb;
            sg.w[i] = *reinterpret_cast<const u32x4 *>(hb + off);
        });
        sg.vlim = r.vlim;
    }
    // DMA: tile r straight into LDS buffer buf, from inside its tile j-1
    // (the buffer's last readers passed the barrier that ended tile j-2).
    // The buffer is eight 1 KiB blocks: K rows 8 b .. 8 b + 7 in block b < 4,
    // V rows 8 (b - 4) on in the others, each block 8 consecutive slots of
    // one page's kv-head block (a half tile is 16 slots of one page). One
    // load per block: lane l lands at byte 16 l of it, as row l / 8, chunk
    // position l % 8, and reads that row's chunk (l % 8) ^ (l / 8) (loff), so
    // row k's chunk c sits at position c ^ (k % 8) and the K and transposed
    // V reads spread over the banks without padding. Rows past the tile's
    // segment end are not loaded and keep finite values (see store). The
    // caller waits (wait_vmcnt0) before the barrier that publishes the tile.
    __device__ __forceinline__ void load_lds(const TileRef &r, uint8_t *buf, uint32_t loff) const
    {
        static_assert(T::DMA, "direct loads: fp16 rows of 64 halves");
        constexpr int W = NTHR / 64;
        const uint32_t P = 1u << log2_page;
        const uint32_t p0 = __builtin_amdgcn_readfirstlane(r.p0), p1 = __builtin_amdgcn_readfirstlane(r.p1);
        const uint8_t *hb0 = pool + ((uint64_t)p0 * page_bytes + head_off);
        const int64_t dhb = ((int64_t)p1 - (int64_t)p0) * (int64_t)page_bytes;
        const int vlim = __builtin_amdgcn_readfirstlane(r.vlim);
        const int lane = tid & 63;
#pragma unroll
        for (int i = 0; i < 8 / W; i++) {
            const int b = wave + W * i;                 // uniform
            const int half = (b >> 1) & 1;
            const uint32_t slot = __builtin_amdgcn_readfirstlane(r.sip0 + (half ? r.dsip : 0u) + 8u * (uint32_t)(b & 1));
            const uint8_t *base = hb0 + (half ? dhb : 0) + (b >= 4 ? P * 128u : 0u) + slot * 128u;
            if (8 * (b & 3) + (lane >> 3) < vlim)
                lds_dma16(base, loff, lds_addr(buf + 1024 * b));
        }
    }
    // A staged tile's chunks into LDS buffer buf. Keys past the tile's
    // segment end (a partial tile: surplus slots of the same pages, whose
    // contents may be anything) must not bring non-finite values, which a
    // zero weight would not remove: fp16 rows there are not stored (ZERO:
    // stored as zeros), so they keep an earlier tile's finite rows or the
    // zeros the buffer starts with; int8 codes are always finite, and their
    // scales there are stored as zeros.
    template <bool ZERO>
    __device__ __forceinline__ void store(const Staged<T::CPT> &sg, uint8_t *buf) const
    {
        const int vlim = sg.vlim;
        const uint32_t P = 1u << log2_page;
        static_for<T::CPT>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            const PfChunk k = pf_chunk<ES, DK, DV, NTHR, i>(tid, wave, P);
            if (k.lds < 0)
                return;
            u32x4 w = sg.w[i];
            if constexpr (ES == 2) {
                if constexpr (ZERO) {
                    if (k.key >= vlim)
                        w = u32x4{0u, 0u, 0u, 0u};
                    *reinterpret_cast<u32x4 *>(buf + k.lds) = w;
                } else if (k.key < vlim) {
                    *reinterpret_cast<u32x4 *>(buf + k.lds) = w;
                }
            } else if (k.scale) {
                if (vlim < PF_KT) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (k.key + e >= vlim)
                            w[e] = 0u;
                }
                *reinterpret_cast<u32x4 *>(buf + k.lds) = w;
            } else {
                *reinterpret_cast<half8 *>(buf + k.lds) = codes8(u32x2{w.x, w.y});
                *reinterpret_cast<half8 *>(buf + k.lds + 16) = codes8(u32x2{w.z, w.w});
            }
        });
    }
};

// 4 waves per SIMD for 8-wave groups and for direct-loaded tiles (no
// staging registers); 3 otherwise (about 160 registers)
template <int ES, int DK, int DV, int REP, int W, bool TAB>
__global__ __launch_bounds__(64 * W)
__attribute__((amdgpu_waves_per_eu(W >= 8 || pf_direct<ES, DK, DV, 64 * W, TAB> ? 4 : 3)))
void prefill_kernel(PrefillArgs a)
{
    using T = PfTile<ES, DK, DV, 64 * W, pf_direct<ES, DK, DV, 64 * W, TAB>>;
    static_assert(DK % 16 == 0 && DV == 64, "prefill tiles: dk multiple of 16, dv 64");
    constexpr int ROWS = 32 * W;
    constexpr int NKB = DK / 16;               // k-blocks of the QK MFMA
    constexpr int NTHR = 64 * W;

    // two tile buffers: one is computed on while the next tile is written
    __shared__ __attribute__((aligned(16))) uint8_t kvbuf[2][T::BUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int jh = lane >> 5, ln = lane & 31;
    // XCD-aware order: work-group w runs on XCD w % 8, so consecutive work
    // items (the row tiles of one sequence and kv-head, which read the same
    // K/V) are given to work-groups of one XCD and share its L2.
    const uint32_t nwg = gridDim.x, wg = blockIdx.x;
    const uint32_t item = (wg % 8u) * (nwg / 8u) + wg / 8u;
    // the work item's record, read-only during the launch (scalar loads)
    const __attribute__((address_space(4))) uint32_t *it =
        (const __attribute__((address_space(4))) uint32_t *)(a.items + 8 * (uint64_t)item);
    const uint32_t seq = it[0];
    if (seq == 0xFFFFFFFFu)
        return;
    const uint32_t g = it[1], rtile = it[2], tok0 = it[3];
    const int ntok = (int)it[4];
    const int pos = (int)it[5];
    const int n_sh = (int)it[6];                // shared-prefix keys (fixed over the chunk)
    const int prefix = (int)it[7];
    const int nrows = ntok * REP;
    const int r0 = (int)rtile * ROWS;

    // this lane's query row
    const int r = r0 + wave * 32 + ln;
    const bool rvalid = r < nrows;
    const int tok = rvalid ? r / REP : 0;
    const int h = (int)g * REP + (rvalid ? r % REP : 0);
    const int qpos = pos + tok;                 // keys [0, qpos] visible
    const uint64_t qrow = (uint64_t)(tok0 + tok) * a.nh + h;

    // rows of this tile: keys up to the last valid row's position
    const int last_r = min(r0 + ROWS, nrows) - 1;
    const int kmax = pos + last_r / REP + 1;        // keys [0, kmax) are touched
    const int kfull = pos + r0 / REP + 1;           // keys [0, kfull) visible to every row

    float16v acc0 = {}, acc1 = {};
    float m = -FLT_MAX, lsum = 0.0f;
    const float neg1 = opaque_neg1();

    PfIO<ES, DK, DV, NTHR, TAB> io;
    io.pool = a.pool;
    io.own_pages = a.page_table + (uint64_t)seq * a.pg.pages_per_seq;
    io.zero = threadIdx.y;
    io.pre_minus_own = prefix >= 0 ? (a.prefix_pages + (uint64_t)prefix * a.pg.pages_per_seq) -
                                         (a.page_table + (uint64_t)seq * a.pg.pages_per_seq) : 0;
    io.head_off = (uint64_t)g * a.pg.head_bytes;
    io.page_bytes = a.pg.page_bytes;
    io.log2_page = a.pg.log2_page;
    io.tid = tid;
    io.wave = __builtin_amdgcn_readfirstlane(wave);
    io.n_sh = n_sh;
    // A shared-prefix decode pass (a.part set) attends the prefix only: its
    // rows are decode queries of sequences attached to it, packed across
    // them, and it leaves each row's softmax state for the sequences' own
    // positions to continue.
    const bool partial = a.part != nullptr;
    io.own_len = partial ? 0 : kmax - n_sh;         // own slots [0, own_len) are touched
    io.nfs = n_sh / PF_KT;
    io.psh = n_sh % PF_KT != 0;
    io.jfull = io.nfs + (partial ? 0 : (kfull - n_sh) / PF_KT);   // + own tiles visible to every row
    io.ntile = io.nfs + io.psh + (io.own_len + PF_KT - 1) / PF_KT;
    const int ntile = io.ntile, jfull = io.jfull;

    // TAB: the tile table (dynamic LDS of a.tab_cap entries, at least every
    // item's tile count), one entry per thread and pass
    if constexpr (TAB) {
        extern __shared__ __attribute__((aligned(16))) uint4 pf_tab[];
        io.tab = pf_tab;
        io.tab_n = (int)min((uint32_t)ntile, a.tab_cap);
        for (int t = tid; t < io.tab_n; t += NTHR) {
            typename PfIO<ES, DK, DV, NTHR, TAB>::TileRef r;
            io.compute(t, r);
            pf_tab[t] = uint4{r.p0, r.p1, r.sip0 | (r.dsip << 16), (uint32_t)r.vlim};
        }
        __syncthreads();
    }

    // Register prefetch: tile j+1 loads while tile j is computed and waits
    // in registers for its LDS store at the end of tile j. The 8-wave
    // variant fits the 128 registers of 4 waves per SIMD; the 2- and 4-wave
    // ones fit 3 waves per SIMD (about 160 registers). A second tile in
    // flight costs those a wave per SIMD and measured slower: a
    // shared-prefix prefill of 48-token suffixes took 0.164 ms at 2 waves
    // per SIMD with two tiles in flight and 0.145 ms at 3 with one. Page ids
    // sit in a ring indexed by tile parity: those of tile j+2 are read at
    // the start of tile j, next to the data load of tile j+1. Tile 0 is
    // requested before Q, so its latency and Q's overlap.
    typename PfIO<ES, DK, DV, NTHR, TAB>::TileRef prn[2];
    Staged<T::CPT> sg;
    // TAB: nxt is the table entry of the tile the next load brings, read
    // before each tile's barrier (whose fence waits for it) and made uniform
    // at the load (DMA: made uniform at once, nref, so that it waits in
    // scalar registers); without a table, page ids sit in a ring indexed by
    // tile parity
    uint4 nxt = {};
    typename PfIO<ES, DK, DV, NTHR, TAB>::TileRef nref = {};
    // DMA: lane's source chunk within a 1 KiB block (see PfIO::load_lds)
    const uint32_t loff = (uint32_t)(lane >> 3) * 128u + 16u * (uint32_t)((lane & 7) ^ (lane >> 3));
    if constexpr (T::DMA) {
        typename PfIO<ES, DK, DV, NTHR, TAB>::TileRef r0;
        if constexpr (TAB) {
            r0 = io.uniform(io.tab[0]);
            nref = io.uniform(io.tab[min(1, io.tab_n - 1)]);
        } else {
            io.fetch(0, prn[0]);
            io.fetch(1, prn[1]);
            r0 = prn[0];
        }
        // buffer 1, and buffer 0's rows past tile 0's segment end (which
        // its load leaves alone), start as zeros (see PfIO::store)
        const int vlim0 = __builtin_amdgcn_readfirstlane(r0.vlim);
        for (int o = tid; o < 2 * T::BUF / 16; o += NTHR)
            if (o >= T::BUF / 16 || ((o >> 3) & (PF_KT - 1)) >= vlim0)
                *reinterpret_cast<u32x4 *>(&kvbuf[0][0] + 16 * o) = u32x4{0u, 0u, 0u, 0u};
        io.load_lds(r0, kvbuf[0], loff);        // tile 0
    } else if constexpr (TAB) {
        io.load(io.uniform(io.tab[0]), sg);     // tile 0
        nxt = io.tab[min(1, io.tab_n - 1)];
    } else {
        io.fetch(0, prn[0]);
        io.fetch(1, prn[1]);
        io.load(prn[0], sg);                    // tile 0
    }
    // Q^T operand, hi and lo halves, slots = dims 16*kb + 8*jh + s: eight
    // consecutive floats per k-block, loaded as two float4 (all issued
    // before any is used; rows past the chunk read row 0 and are zeroed).
    half8 qh[NKB], ql[NKB];
    {
        const float *qr = a.q + (rvalid ? qrow : (uint64_t)tok0 * a.nh + (int)g * REP) * DK + 8 * jh;
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
            u32x4 hw, lw;
#pragma unroll
            for (int s = 0; s < 8; s += 2) {
                // hi (rounded toward zero, two per conversion) and lo = x -
                // hi rounded to nearest, as for P. Both must derive from the
                // one rounded fp32 x: the empty asm keeps the compiler from
                // feeding either conversion the exact product (a fused
                // multiply-convert), which would pair lo with another hi.
                float x0 = xs[s] * qs, x1 = xs[s + 1] * qs;
                asm volatile("" : "+v"(x0), "+v"(x1));
                const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
                hw[s >> 1] = h;
                lw[s >> 1] = split_lo2(h, x0, x1, neg1);
            }
            qh[kb] = __builtin_bit_cast(half8, hw);
            ql[kb] = __builtin_bit_cast(half8, lw);
        }
    }

    if constexpr (T::DMA) {
        wait_vmcnt0();
    } else {
        io.template store<true>(sg, kvbuf[0]);
        if constexpr (ES == 2) {
            // the other buffer starts as zeros (see PfIO::store)
            for (int o = 16 * tid; o < T::BUF; o += 16 * NTHR)
                *reinterpret_cast<u32x4 *>(kvbuf[1] + o) = u32x4{0u, 0u, 0u, 0u};
        }
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
        // the data of tile j+1 (past the last tile: the last tile again,
        // never stored); without a table, first the ids of tile j+2 into the
        // slot of tile j's (spent)
        if constexpr (T::DMA) {
            if constexpr (!TAB)
                io.fetch(j + 2, prn[PJ]);
            if (j + 1 < ntile)
                io.load_lds(TAB ? nref : prn[Q1], kvbuf[Q1], loff);
        } else if constexpr (TAB) {
            io.load(io.uniform(nxt), sg);
        } else {
            io.fetch(j + 2, prn[PJ]);
            io.load(prn[Q1], sg);
        }
        const _Float16 (*Ks)[T::KPAD] = reinterpret_cast<const _Float16 (*)[T::KPAD]>(kvbuf[PJ]);
        const _Float16 (*Vr)[T::VPAD] = reinterpret_cast<const _Float16 (*)[T::VPAD]>(kvbuf[PJ] + T::VOFF);
        const float *Ksc = reinterpret_cast<const float *>(kvbuf[PJ] + T::SOFF), *Vsc = Ksc + PF_KT;

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
            const half8 ka = T::DMA ? *reinterpret_cast<const half8 *>(kvbuf[PJ] + ln * 128 + 16 * ((2 * kb + jh) ^ (ln & 7)))
                                    : *reinterpret_cast<const half8 *>(&Ks[ln][16 * kb + 8 * jh]);
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
            // key kl of the tile is position tb + kl, visible up to lim:
            // register i (key 8 (i / 4) + 4 jh + i % 4) is masked when
            // 8 (i / 4) + i % 4 > lim - tb - 4 jh
            bool sh;
            int s0, len;
            io.seg(j, sh, s0, len);
            const int tb = sh ? s0 : n_sh + s0, lim = sh ? n_sh - 1 : qpos;
            const int thr = lim - tb - 4 * jh;
#pragma unroll
            for (int i = 0; i < 16; i++)
                st[i] = 8 * (i >> 2) + (i & 3) > thr ? -INFINITY : st[i];
        }
        // Lazy max (below): the running max moves only when a score exceeds
        // it by more than 2^8, so weights stay <= 256 (exact range for fp16
        // and fp32). With fp16 K/V, after the first tile, that is checked on
        // the weights instead of the scores: each 16-key half's exps are
        // summed for the row sum anyway, and a half whose sum is at most 256
        // holds no weight above 256, so the tile max is needed only when a
        // sum exceeds it (rare once the running max has settled). Otherwise
        // the tile max decides first.
        constexpr bool SUMCHK = REL;
        if constexpr (!SUMCHK) {
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
        }
        // P^T operand (hi, lo) and O^T += V^T . P^T, one 16-key block at a
        // time (keys 16*kb2 + 8*(s/4) + 4*jh + (s%4) in slot s): a block's
        // weights are made just before its MFMAs, which keeps their live
        // ranges short. hi = p rounded toward zero to fp16, lo = the remainder.
#pragma unroll
        for (int kb2 = 0; kb2 < 2; kb2++) {
            float p[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                p[i] = fast_exp2(REL ? st[8 * kb2 + i] : st[8 * kb2 + i] - m);
            if constexpr (SUMCHK) {
                float ts = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                if (__builtin_expect(__ballot(ts > 256.0f) != 0, 0)) {
                    // the half's max over the row (this lane's 8 keys and its
                    // partner's), then the running max moves as above; the
                    // other half's scores move with it
                    const float h0 = max3(st[8 * kb2], st[8 * kb2 + 1], st[8 * kb2 + 2]);
                    const float h1 = max3(st[8 * kb2 + 3], st[8 * kb2 + 4], st[8 * kb2 + 5]);
                    float mt = max3(h0, h1, __builtin_fmaxf(st[8 * kb2 + 6], st[8 * kb2 + 7]));
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
                    mt = max3(mt, __uint_as_float(sw[0]), __uint_as_float(sw[1]));
                    const bool grow = mt > 8.0f;
                    if (__ballot(grow) != 0) {
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
#pragma unroll
                        for (int i = 0; i < 8; i++)
                            p[i] = fast_exp2(st[8 * kb2 + i]);
                        ts = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                    }
                }
                lsum += ts;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i += 2)
                    lsum += p[i] + p[i + 1];
            }
            u32x4 phw, plw;
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                float p0 = p[i], p1 = p[i + 1];
                if constexpr (ES == 1) {
                    p0 *= Vsc[8 * ((8 * kb2 + i) >> 2) + 4 * jh + (i & 3)];
                    p1 *= Vsc[8 * ((8 * kb2 + i) >> 2) + 4 * jh + ((i + 1) & 3)];
                }
                const fp16x2 h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
                const uint32_t hw = __builtin_bit_cast(uint32_t, h);
                phw[i >> 1] = hw;
                plw[i >> 1] = split_lo2(hw, p0, p1, neg1);
            }
            const half8 ph = __builtin_bit_cast(half8, phw), pl = __builtin_bit_cast(half8, plw);
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                // V^T rows 32 dt + ln, keys 16 kb2 + 4 jh + [0, 4) and 8 on:
                // in each 16-lane group ds_read_b64_tr_b16 gives output lane i
                // element j from the address of lane 4 j + i / 4 (plus i % 4),
                // so lane (j, q) of the group points at key j, dims 4 q on
                // (DMA: row k's 16-byte chunk c at position c ^ (k % 8), the
                // same for the rows 8 on)
                const int vk = 16 * kb2 + 4 * jh + ((lane >> 2) & 3);
                const int vc = 4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
                const _Float16 *vr = T::DMA ? reinterpret_cast<const _Float16 *>(kvbuf[PJ] + T::VOFF + vk * 128 + 16 * (vc ^ (vk & 7)) + 8 * (lane & 1))
                                            : &Vr[vk][32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)];
                const half4 v0 = tr16_read(vr);
                const half4 v1 = tr16_read(vr + (T::DMA ? 8 * 64 : 8 * T::VPAD));
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
        if constexpr (T::DMA)
            wait_vmcnt0();       // tile j+1's direct loads have landed
        else if (j + 1 < ntile)  // tile j+1 into the other buffer (its readers are done)
            io.template store<false>(sg, kvbuf[Q1]);
        if constexpr (TAB && T::DMA)
            nref = io.uniform(io.tab[min(j + 2, io.tab_n - 1)]);
        else if constexpr (TAB)
            nxt = io.tab[min(j + 2, io.tab_n - 1)];
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
    // the row's output index and lane half again, from an opaque copy of the
    // thread id: held across the tiles, they were spilled (DMA variants)
    uint64_t qrow_e = qrow;
    int jh_e = jh;
    if constexpr (T::DMA) {
        int te = tid;
        asm volatile("" : "+v"(te));
        const int re = r0 + (te >> 6) * 32 + (te & 31);
        qrow_e = (uint64_t)(tok0 + re / REP) * a.nh + (int)g * REP + re % REP;
        jh_e = (te >> 5) & 1;
    }
    if (partial) {
        // split-KV chunk 0 of the row: unnormalised sums, the running max
        // (base 2) and the sum of weights, as the decode kernel's partials
        float *pr = a.part + qrow_e * a.max_chunks * (DV + 2);
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
            const float16v &acc = dt == 0 ? acc0 : acc1;
#pragma unroll
            for (int i = 0; i < 16; i++)
                pr[32 * dt + 8 * (i >> 2) + 4 * jh_e + (i & 3)] = acc[i];
        }
        if (jh_e == 0) {
            pr[DV] = m;
            pr[DV + 1] = lsum;
        }
        return;
    }
    const float inv = 1.0f / lsum;
    float *o = a.out + qrow_e * DV;
    const float *gt = a.gate ? a.gate + qrow_e * DV : nullptr;
#pragma unroll
    for (int dt = 0; dt < 2; dt++) {
#pragma unroll
        for (int i4 = 0; i4 < 4; i4++) {
            const int d0 = 32 * dt + 8 * i4 + 4 * jh_e;
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
// group's rep query heads as the wave's columns (16 slots, rep of them
// valid), every visible slot as its keys, in slot order (sinks, shared
// prefix and ring alike; softmax does not depend on the order, and the
// visible set is the engine's, engine/src/nd_model.c:2451-2483). Per 32-key
// tile:
//   S^T[32 keys x 16 cols]  = K . Q^T          v_mfma_f32_16x16x32_f16
//   O^T[64 dims x 16 cols] += V^T . P^T
// Q and P are fp16 hi + lo pairs (two MFMAs each): fp32-level accuracy, as in
// the prefill kernel; the lazy running max likewise.
//
// K/V stay int8 codes in LDS, written raw with 16-byte stores from the
// registers a tile was loaded into, and become fp16 as they are read into an
// operand: one xor, two byte permutes and two packed fp16 subtracts per four
// codes (0x64 over the byte code ^ 0x80 is the fp16 1024 + code + 128). V^T
// comes out of row-major V with ds_read_b64_tr_b8 (in each 16-lane group,
// output lane i byte j is byte i % 8 at the address of lane 2 j + i / 8). The
// k scale multiplies S and the v scale folds into P: the engine's
// dequantisation (engine/src/nd_model.c:2179-2180, :2250-2252).
// four int8 codes as the low k slots of an operand whose upper four are zero
__device__ __forceinline__ half8 codes4(uint32_t w)
{
    const uint32_t x = w ^ 0x80808080u;
    const half2v c0 = codes2<0x04010400>(x), c1 = codes2<0x04030402>(x);
    return half8{c0[0], c0[1], c1[0], c1[1], 0, 0, 0, 0};
}

typedef float float4v __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

__device__ __forceinline__ float4v mfma16k32(half8 a, half8 b, float4v c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Lane layouts (16 x 16 tiles): lane l = 16 g + r holds MFMA row / column r
// and the k (or output row) slots of lane group g. Row r of S block kb reads
// key 8 (r / 4) + 4 kb + r % 4, so the S^T rows lane (r, g) receives are keys
// 8 g + 4 kb + i: its eight scores are keys 8 g .. 8 g + 7 in order, which is
// the k-slot order of the P^T operand, and V^T is read for the same keys.
// A column's softmax state spans the four lane groups (a max and a sum
// across them).
//
// Tiles are 32 slots of one segment (the shared prefix's pages, then the
// sequence's own), aligned to 32 within it, so a tile's keys 16 h .. 16 h + 15
// are consecutive slots of one page: per half tile, one load each reads its
// K rows, V rows and scales, contiguous runs of the page (every cache line
// requested once). A segment's last tile can be partial: its surplus keys
// read slots of the same pages (or half 0 again) and are masked.
//
// A wave keeps one tile in flight in registers (loaded while the previous
// one is computed) and one in its LDS buffer. Splitting a row's tiles over
// more waves (and merging their states) measured no faster: the launch is
// bound by its memory stream, not by the wave count.
//
// RUN (pages of 16 slots, K + V + scales of a kv-head within 128 chunks of
// 16 bytes): a half tile is a whole kv-head block of one page, 1920 bytes at
// qk 48, read as one contiguous run by two loads.
template <int DK, int DV, int REP, bool RUN>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4)))
void decode_mfma_kernel(PrefillArgs a)
{
    static_assert(DK % 16 == 0 && DK <= 64 && DV == 64 && REP <= 16,
                  "decode tiles: dk multiple of 16 up to 64, dv 64, rep <= 16");
    static_assert(!RUN || DK + DV + 8 <= 128, "a kv-head block of a 16-slot page within two loads");
    constexpr int NS = DK / 32;                 // 32-dim steps of S (16x16x32)
    // A last 16-dim step (qk 48) runs on the same 16x16x32 instruction, its
    // upper four k slots zero in both operands. Every accumulation chain
    // thus keeps one opcode: an MFMA reading as its accumulator the result
    // of the MFMA issued just before it, of another opcode (16x16x16 after
    // 16x16x32), gave wrong results on gfx950 although the compiler puts no
    // wait state between them, as it does for the same opcode.
    constexpr bool TAIL = DK % 32 == 16;
    constexpr int VSTR = DV + 16;               // V row stride: spreads the transposed reads over the banks
    constexpr int KB = PF_KT * DK, VB = PF_KT * VSTR;
    __shared__ __attribute__((aligned(16))) uint8_t lds[KB + VB + PF_KT * 8];   // K, V, k scales, v scales

    const int lane = threadIdx.x;
    const int g = lane >> 4, r = lane & 15;     // MFMA: lane group, row / column
    const uint32_t nkv = a.pg.nkv;
    // a.items: the rows' work order (longest first), or null: in order
    const uint32_t b = a.items ? *(const __attribute__((address_space(4))) uint32_t *)(a.items + blockIdx.x / nkv)
                               : blockIdx.x / nkv;
    const uint32_t kvh = blockIdx.x % nkv;
    // row ids, sequence state and page tables are read-only during the
    // launch and uniform per wave: read through the constant address space
    // (scalar loads)
    const uint32_t seq = a.row_seq ? *(const __attribute__((address_space(4))) uint32_t *)(a.row_seq + b) : b;
    SeqDev sd;
    {
        const cptr sp = (cptr)(a.seqs + seq);
        sd.pos = sp[0];
        sd.n_sink = sp[1];
        sd.prefix = sp[2];
    }
    const Visible vis = visible(sd, sd.pos, (int)a.pg.window);
    const int n_sh = vis.n_sh, n_own = vis.n_own;

    // Load plan of a half tile (16 keys), per lane: K chunk c = lane % DK (16
    // bytes; with qk 48 lanes 48..63 repeat chunks 0..15: same data, same LDS
    // bytes), V chunk `lane`, and scale word `lane % 32` (16 k scales, then
    // 16 v scales). Offsets are from the kv-head block of the half's page;
    // the half's first slot adds sip * DK, sip * DV and sip * 4.
    // RUN: 16-byte chunks `lane` and 64 + lane of the block (K rows, V rows,
    // k scales, v scales; surplus lanes repeat the last chunk), each with its
    // LDS place per half.
    const int P = 1 << a.pg.log2_page;
    constexpr int NRC = DK + DV + 8;           // chunks of a 16-slot kv-head block
    auto run_lds = [&](int c, int h) __attribute__((always_inline)) -> int {
        if (c < DK)
            return 16 * DK * h + 16 * c;
        if (c < DK + DV)
            return KB + (16 * h + (c - DK) / 4) * VSTR + 16 * ((c - DK) % 4);
        const int sc = c - DK - DV;
        return KB + VB + 128 * (sc >> 2) + 64 * h + 16 * (sc & 3);
    };
    const int rc1 = min(64 + lane, NRC - 1);
    const uint32_t rg1 = 16 * rc1;
    // RUN: the first slot a chunk holds (K rows, V rows, then 4 slots of k
    // or v scales per chunk); a chunk whose slots are all past the half's
    // visible ones is not fetched (its lane reads chunk 0 instead, one line
    // for the wave): the keys it would feed are masked
    auto run_slot = [&](int c) __attribute__((always_inline)) -> int {
        if (c < DK)
            return c * 16 / DK;
        if (c < DK + DV)
            return (c - DK) * 16 / DV;
        return 4 * ((c - DK - DV) & 3);
    };
    const int rs0 = run_slot(lane), rs1 = run_slot(rc1);
    int rl[2][2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        rl[h][0] = run_lds(lane, h);
        rl[h][1] = run_lds(rc1, h);
    }
    const uint32_t kc = 16 * (lane % DK);
    const uint32_t gv = P * DK + 16 * lane;
    const int lv = KB + (lane >> 2) * VSTR + 16 * (lane & 3);
    const int sw = lane & 31, which = sw >> 4;
    const uint32_t gs = P * (DK + DV) + which * 4 * P + 4 * (sw & 15);
    const int ls = KB + VB + 128 * which + 4 * (sw & 15);

    const cptr own = (cptr)(a.page_table + (uint64_t)seq * a.pg.pages_per_seq);
    const cptr pre = sd.prefix >= 0 ? (cptr)(a.prefix_pages + (uint64_t)sd.prefix * a.pg.pages_per_seq) : own;
    const int tiles_sh = (n_sh + PF_KT - 1) / PF_KT;
    const int ntile = tiles_sh + (n_own + PF_KT - 1) / PF_KT;
    // tile j: its segment's visible slots from its first on
    auto remaining = [&](int j) __attribute__((always_inline)) {
        return j < tiles_sh ? n_sh - PF_KT * j : n_own - PF_KT * (j - tiles_sh);
    };
    // tile j: page ids and first in-page slots of its halves (half 1 past
    // the segment's end rereads half 0)
    struct TileRef {
        int32_t pid[2];
        int sip[2], vis[2];                     // vis: the half's visible slots (RUN)
    };
    auto fetch = [&](int j, TileRef &tr_) __attribute__((always_inline)) {
        j = min(j, ntile - 1);
        const bool sh = j < tiles_sh;
        const int s0 = PF_KT * (sh ? j : j - tiles_sh);
        const int len = sh ? n_sh : n_own;
        const cptr rows = sh ? pre : own;
        const int s1 = s0 + 16 < len ? s0 + 16 : s0;
        tr_.pid[0] = rows[s0 >> a.pg.log2_page];
        tr_.pid[1] = rows[s1 >> a.pg.log2_page];
        tr_.sip[0] = s0 & (P - 1);
        tr_.sip[1] = s1 & (P - 1);
        tr_.vis[0] = min(16, len - s0);
        tr_.vis[1] = s1 != s0 ? min(16, len - s1) : 0;
    };
    struct Stage {
        u32x4 k[2], v[2];                       // RUN: chunks lane and 64 + lane
        float sc[2];
    };
    auto load = [&](const TileRef &t_, Stage &sg) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // a page is under 4 GiB: one 32 x 32 -> 64-bit multiply-add
            const uint8_t *hb = a.pool + (uint64_t)(uint32_t)t_.pid[h] * (uint32_t)a.pg.page_bytes +
                                (uint64_t)kvh * a.pg.head_bytes;
            if constexpr (RUN) {
                const uint32_t o0 = rs0 < t_.vis[h] ? 16 * lane : 0u, o1 = rs1 < t_.vis[h] ? rg1 : 0u;
                sg.k[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(hb + o0));
                sg.v[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(hb + o1));
            } else {
                const uint32_t sip = (uint32_t)t_.sip[h];
                sg.k[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(hb + (kc + sip * DK)));
                sg.v[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(hb + (gv + sip * DV)));
                sg.sc[h] = __builtin_nontemporal_load(reinterpret_cast<const float *>(hb + (gs + sip * 4)));
            }
        }
    };
    auto store = [&](const Stage &sg) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if constexpr (RUN) {
                *reinterpret_cast<u32x4 *>(lds + rl[h][0]) = sg.k[h];
                *reinterpret_cast<u32x4 *>(lds + rl[h][1]) = sg.v[h];
                continue;
            }
            *reinterpret_cast<u32x4 *>(lds + kc + 16 * DK * h) = sg.k[h];
            *reinterpret_cast<u32x4 *>(lds + lv + 16 * VSTR * h) = sg.v[h];
            *reinterpret_cast<float *>(lds + ls + 64 * h) = sg.sc[h];
        }
    };

    // the first tile goes out before the q loads, so that their latencies
    // overlap; tref then holds the references of the next tile
    TileRef tref;
    Stage sg;
    fetch(0, tref);
    load(tref, sg);
    fetch(1, tref);

    // Q^T operand, hi and lo: column r, dims 32 s + 8 g + [0, 8) and the tail
    // 32 NS + 4 g + [0, 4) (then four zero slots); hi and lo from one rounded
    // fp32 value
    const bool rvalid = r < REP;
    const uint64_t qrow = (uint64_t)b * a.nh + kvh * REP + (rvalid ? r : 0);
    half8 qh[NS + TAIL], ql[NS + TAIL];
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
            qh[NS] = half8{};
            ql[NS] = half8{};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                _Float16 hi, lo;
                split(xs[i], hi, lo);
                qh[NS][i] = hi;
                ql[NS][i] = lo;
            }
        }
    }

    // lane-constant LDS offsets: the S operand rows (block 0; block 1 is 4
    // rows on), the V^T rows (dims 0..15), the k scales of the keys whose
    // scores this lane holds (v scales 128 bytes on)
    const int koff = (8 * (r >> 2) + (r & 3)) * DK;
    const int voff = KB + (8 * g + (r >> 1)) * VSTR + 8 * (r & 1);
    const int soff = KB + VB + 32 * g;

    float4v acc[4] = {};                        // O^T: dims 16 d + 4 g + i, column r
    float m = -FLT_MAX, lsum = 0.0f;
    const float neg1 = opaque_neg1();

    // the gate of this lane's output dims 16 d + 4 g + [0, 4), loaded with
    // the last tile's arithmetic, so that its latency does not end the wave
    const float *gt = a.gate ? a.gate + qrow * DV : nullptr;
    float4 gv4[4];

    // tile j: the load of the next tile (references fetched a tile ago), the
    // references of the one after, the tile's arithmetic, then the next tile
    // into LDS; the last tile loads the gate instead
    // Scores are kept relative to the running max m: after the first tile
    // (which sets m to its own max), one fma per score applies the k scale
    // and subtracts m, and the lazy check compares with 8 alone.
    auto tile = [&](const int j, auto masked, auto last, auto first) __attribute__((always_inline)) {
        constexpr bool more = !decltype(last)::value;
        constexpr bool FIRST = decltype(first)::value;
        const int rem = remaining(j) - 8 * g;   // this lane's visible keys of the tile
        if constexpr (more) {
            load(tref, sg);
            fetch(j + 2, tref);
        } else {
#pragma unroll
            for (int d = 0; d < 4; d++)
                gv4[d] = gt && rvalid ? *reinterpret_cast<const float4 *>(gt + 16 * d + 4 * g) : float4{0, 0, 0, 0};
        }

        float4v st[2];
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const uint8_t *kr = lds + koff + kb * 4 * DK;
            st[kb] = float4v{};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const half8 ka = codes8(*reinterpret_cast<const u32x2 *>(kr + 32 * s + 8 * g));
                st[kb] = mfma16k32(ka, qh[s], st[kb]);
                st[kb] = mfma16k32(ka, ql[s], st[kb]);
            }
            if constexpr (TAIL) {
                const half8 ka = codes4(*reinterpret_cast<const uint32_t *>(kr + 32 * NS + 4 * g));
                st[kb] = mfma16k32(ka, qh[NS], st[kb]);
                st[kb] = mfma16k32(ka, ql[NS], st[kb]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        // scores of keys 8 g + 4 kb + i: k scales, then the mask (a masked
        // key's v scale, possibly never written, becomes 0)
        float vsc[8];
        const float nm = -m;
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const float4 ks = *reinterpret_cast<const float4 *>(lds + soff + 16 * kb);
            const float4 vs = *reinterpret_cast<const float4 *>(lds + soff + 128 + 16 * kb);
            if constexpr (FIRST) {
                st[kb] *= float4v{ks.x, ks.y, ks.z, ks.w};
            } else {
                st[kb][0] = __builtin_fmaf(st[kb][0], ks.x, nm);
                st[kb][1] = __builtin_fmaf(st[kb][1], ks.y, nm);
                st[kb][2] = __builtin_fmaf(st[kb][2], ks.z, nm);
                st[kb][3] = __builtin_fmaf(st[kb][3], ks.w, nm);
            }
            vsc[4 * kb + 0] = vs.x;
            vsc[4 * kb + 1] = vs.y;
            vsc[4 * kb + 2] = vs.z;
            vsc[4 * kb + 3] = vs.w;
        }
        if constexpr (decltype(masked)::value) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const bool out = 4 * kb + i >= rem;
                    st[kb][i] = out ? -INFINITY : st[kb][i];
                    vsc[4 * kb + i] = out ? 0.0f : vsc[4 * kb + i];
                }
        }
        // the column's tile max over its 32 keys: 8 in this lane, then across
        // the four lane groups (lanes r + 16 g)
        const float y0 = max3(st[0][0], st[0][1], st[0][2]), y1 = max3(st[0][3], st[1][0], st[1][1]);
        float mt = max3(y0, y1, max3(st[1][2], st[1][3], st[1][3]));
        mt = max3(mt, __shfl_xor(mt, 16, 64), mt);
        {
            const auto sw2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = max3(mt, __uint_as_float(sw2[0]), __uint_as_float(sw2[1]));
        }
        if constexpr (FIRST) {
            // the first tile sets m (nothing is accumulated yet)
            m = mt;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
                st[kb] -= mt;
        } else {
            // scores relative to m: it moves only when one exceeds it by 2^8
            const bool grow = mt > 8.0f;
            if (__builtin_expect(__ballot(grow) != 0, 0)) {
                const float d = grow ? mt : 0.0f;
                const float rs = fast_exp2(-d);
                m += d;
                lsum *= rs;
#pragma unroll
                for (int dd = 0; dd < 4; dd++)
                    acc[dd] *= rs;
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
                    st[kb] -= d;
            }
        }
        float p[8];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                p[4 * kb + i] = fast_exp2(st[kb][i]);
        lsum += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
#pragma unroll
        for (int i = 0; i < 8; i++)
            p[i] *= vsc[i];
        // P^T operand (hi, lo): slots = keys 8 g .. 8 g + 7; hi = p rounded
        // toward zero to fp16, lo = the remainder
        u32x4 phw, plw;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const fp16x2 hh = __builtin_amdgcn_cvt_pkrtz(p[i], p[i + 1]);
            const uint32_t hw = __builtin_bit_cast(uint32_t, hh);
            phw[i >> 1] = hw;
            plw[i >> 1] = split_lo2(hw, p[i], p[i + 1], neg1);
        }
        const half8 ph = __builtin_bit_cast(half8, phw), pl = __builtin_bit_cast(half8, plw);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const v2i w = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_v2i *)(__attribute__((address_space(3))) void *)(lds + voff + 16 * d));
            const half8 va = codes8(u32x2{(uint32_t)w.x, (uint32_t)w.y});
            acc[d] = mfma16k32(va, ph, acc[d]);
            acc[d] = mfma16k32(va, pl, acc[d]);
        }
        __builtin_amdgcn_s_setprio(0);
        // The next tile into LDS after this tile's last LDS reads. Other lanes
        // of the wave read what this lane stores, and the wave's LDS accesses
        // complete in issue order; the wave barriers (scheduling barriers,
        // no instruction) keep the compiler from moving LDS accesses of one
        // tile across the store of the next.
        if constexpr (more) {
            __builtin_amdgcn_wave_barrier();
            store(sg);
            __builtin_amdgcn_wave_barrier();
        }
    };
    store(sg);
    using Yes = std::true_type;
    using No = std::false_type;
    if (ntile == 1) {
        if (remaining(0) >= PF_KT)
            tile(0, No{}, Yes{}, Yes{});
        else
            tile(0, Yes{}, Yes{}, Yes{});
    } else {
        if (remaining(0) >= PF_KT)
            tile(0, No{}, No{}, Yes{});
        else
            tile(0, Yes{}, No{}, Yes{});
        for (int j = 1; j + 1 < ntile; j++) {
            if (remaining(j) >= PF_KT)
                tile(j, No{}, No{}, No{});
            else
                tile(j, Yes{}, No{}, No{});
        }
        if (remaining(ntile - 1) >= PF_KT)
            tile(ntile - 1, No{}, Yes{}, No{});
        else
            tile(ntile - 1, Yes{}, Yes{}, No{});
    }

    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    if (!rvalid)
        return;
    const float inv = 1.0f / lsum;
    float *o = a.out + qrow * DV;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const int d0 = 16 * d + 4 * g;
        float4 z;
        z.x = acc[d][0] * inv;
        z.y = acc[d][1] * inv;
        z.z = acc[d][2] * inv;
        z.w = acc[d][3] * inv;
        if (gt) {
            z.x *= sigmoid_dev(gv4[d].x);
            z.y *= sigmoid_dev(gv4[d].y);
            z.z *= sigmoid_dev(gv4[d].z);
            z.w *= sigmoid_dev(gv4[d].w);
        }
        // streamed past L2 (like the K/V loads): the output is not read
        // again in this launch, and plain stores took 4.5% longer (60.7-61.0
        // against 57.9-58.1 us per 4096-row launch, back to back)
        __builtin_nontemporal_store(float4v{z.x, z.y, z.z, z.w}, reinterpret_cast<float4v *>(o + d0));
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
    const bool p16 = a.pg.log2_page == 4;
#define X(DK, DV, REP)                                                                                  \
    if (!g.kv_f16 && g.dk == DK && g.dv == DV && g.rep == REP) {                                        \
        if (p16 && DK + DV + 8 <= 128)                                                                  \
            hipLaunchKernelGGL((decode_mfma_kernel<DK, DV, REP, (DK + DV + 8 <= 128)>), dim3(a.n_items), \
                               dim3(64), 0, s, a);                                                      \
        else                                                                                            \
            hipLaunchKernelGGL((decode_mfma_kernel<DK, DV, REP, false>), dim3(a.n_items), dim3(64), 0, s, a); \
        return hipGetLastError();                                                                       \
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

template <int ES, int DK, int DV, int REP, bool TAB>
static void launch_pf(dim3 grid, int waves, uint32_t lds, const PrefillArgs &a, hipStream_t s)
{
    if (waves == 2)
        hipLaunchKernelGGL((prefill_kernel<ES, DK, DV, REP, 2, TAB>), grid, dim3(128), lds, s, a);
    else if (waves == 8)
        hipLaunchKernelGGL((prefill_kernel<ES, DK, DV, REP, 8, TAB>), grid, dim3(512), lds, s, a);
    else
        hipLaunchKernelGGL((prefill_kernel<ES, DK, DV, REP, 4, TAB>), grid, dim3(256), lds, s, a);
}

// Largest tile table (bytes of dynamic LDS) that keeps a work-group size's
// residency: 160 KiB per CU over its resident work-groups, less two tile
// buffers. 8-wave groups and the 2- and 4-wave ones with direct-loaded
// tiles (dma: fp16, qk 64; 16 KiB of buffers) run 4 waves per SIMD; the
// others 3. Staged buffers take at most 19 KiB.
uint32_t pf_tab_max_bytes(int waves, bool dma)
{
    if (waves >= 8)
        return 48u << 10;   // staged tiles: 19 KiB of buffers
    if (dma)
        return waves == 4 ? 22u << 10 : 3584u;
    return waves == 4 ? 32u << 10 : 7u << 10;
}

hipError_t launch_prefill(const Geo &g, const PrefillArgs &a, int waves, hipStream_t s)
{
    if (a.n_items == 0)
        return hipSuccess;
    if (waves == 8 && !pf_w8_fits(g))
        waves = 4;
    const int es = g.kv_f16 ? 2 : 1;
    dim3 grid(a.n_items);     // n_items: a multiple of 8 (padded with empty items)
    // a table of a.tab_cap tiles when the host sized one that fits
    const uint32_t tab_bytes = a.tab_cap * 16u;
    const bool tab = a.tab_cap > 0 && tab_bytes <= pf_tab_max_bytes(waves, es == 2 && g.dk == 64 && g.dv == 64);
#define X(ES, DK, DV, REP)                                                                      \
    if (es == ES && g.dk == DK && g.dv == DV && g.rep == REP) {                                 \
        if (tab)                                                                                 \
            launch_pf<ES, DK, DV, REP, true>(grid, waves, tab_bytes, a, s);                      \
        else                                                                                     \
            launch_pf<ES, DK, DV, REP, false>(grid, waves, 0, a, s);                             \
        return hipGetLastError();                                                                \
    }
    NDA_PF_GEOMETRIES(X)
#undef X
    return hipErrorNotSupported;
}

} // namespace nda
