// nda_kernels.hip - gfx950 kernels of the Needle attention / KV-cache path.
//
// Decode attention (attend_kernel) is HBM-bound: every K/V byte is read once.
// A work-group of NW waves owns one (row, kv-head) unit (a row is one query
// token of one sequence) or one split-KV chunk of it. Inside a wave, G lanes
// share one KV position: each lane loads its 16-byte slice of the K and V row
// straight into registers (global_load_dwordx4, a wave moves 1 KiB per load)
// and 64/G positions are in flight per wave per step. The q.k partial dots
// are summed over the G lanes with DPP row permutes; every lane group keeps
// its own online-softmax state (running max, denominator, accumulator), so no
// wave-wide reduction happens inside the KV loop. The states are merged once
// at the end (shuffles across lane groups, LDS across waves). With no reuse
// of K/V rows between lanes (rep 1) there is nothing to gain from staging
// K/V in LDS; for GQA the rep query heads of a group reuse each loaded row
// from registers.
//
// Semantics follow the engine's attn_heads (engine/src/nd_model.c:2105-2359):
// the visited positions are the sinks plus the recent ring (:2451-2483), the
// current token included, emit (acc / denom) * sigmoid(gate) (:2085-2103).
// The online softmax is evaluated in base 2 (q pre-scaled by log2(e)/sqrt(dk))
// with fp32 accumulation; results match the engine's fp32 CPU attention to
// rounding (tests bound max |delta| at 1e-3).
#include "nda_device.h"

#include <float.h>

namespace nda {

// ---------------------------------------------------------------- helpers

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes; every lane of a group gets the same
// bits (each step adds a commutative pair).
template <int G>
__device__ __forceinline__ float group_sum(float x)
{
    if constexpr (G >= 2)
        x += dpp_mov<0xB1>(x);    // quad_perm [1,0,3,2]
    if constexpr (G >= 4)
        x += dpp_mov<0x4E>(x);    // quad_perm [2,3,0,1]
    if constexpr (G >= 8)
        x += dpp_mov<0x141>(x);   // row_half_mirror
    if constexpr (G >= 16)
        x += dpp_mov<0x140>(x);   // row_mirror
    static_assert(G <= 16, "group_sum: G <= 16");
    return x;
}

// ----------------------------------------------------- fixed-size loads

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int NB>
struct Words {
    static_assert(NB % 4 == 0, "row slices are whole dwords");
    uint32_t w[NB / 4];
};

// NT: nontemporal loads (a row read once); plain loads where other
// work-groups read the same rows (a shared prefix), which L2 then keeps
template <typename V, bool NT>
__device__ __forceinline__ V ld(const V *p)
{
    if constexpr (NT)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

template <int NB, bool NT = true>
__device__ __forceinline__ void load_words(Words<NB> &d, const uint8_t *p)
{
    if constexpr (NB % 16 == 0) {
#pragma unroll
        for (int i = 0; i < NB / 16; i++) {
            u32x4 x = ld<u32x4, NT>(reinterpret_cast<const u32x4 *>(p) + i);
            d.w[4 * i + 0] = x.x;
            d.w[4 * i + 1] = x.y;
            d.w[4 * i + 2] = x.z;
            d.w[4 * i + 3] = x.w;
        }
    } else if constexpr (NB % 8 == 0) {
#pragma unroll
        for (int i = 0; i < NB / 8; i++) {
            u32x2 x = ld<u32x2, NT>(reinterpret_cast<const u32x2 *>(p) + i);
            d.w[2 * i + 0] = x.x;
            d.w[2 * i + 1] = x.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NB / 4; i++)
            d.w[i] = ld<uint32_t, NT>(reinterpret_cast<const uint32_t *>(p) + i);
    }
}

// The first nb bytes of a slice (whole dwords; nb may be <= 0), the rest zero:
// a lane's part of a row whose true length is shorter than the padded one.
template <int NB, bool NT = true>
__device__ __forceinline__ void load_words_upto(Words<NB> &d, const uint8_t *p, int nb)
{
#pragma unroll
    for (int i = 0; i < NB / 4; i++)
        d.w[i] = 4 * i < nb ? ld<uint32_t, NT>(reinterpret_cast<const uint32_t *>(p) + i) : 0u;
}

// Element e of a loaded slice as float: int8 code or fp16 value.
template <int ES>
__device__ __forceinline__ float elem(const uint32_t *w, int e)
{
    if constexpr (ES == 1) {
        return (float)(int8_t)(w[e >> 2] >> (8 * (e & 3)));
    } else {
        uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        return (float)__builtin_bit_cast(_Float16, h);
    }
}

// -------------------------------------------------------- decode / causal

template <int ES, int DK, int DV, int REP, int G, int NP, int NW>
struct AttnCfg {
    static constexpr int EK = DK / G;          // K elements per lane
    static constexpr int EV = DV / G;          // V elements per lane
    static constexpr int PW = 64 / G;          // positions per wave step (lane groups)
    static constexpr int KB = EK * ES;         // K bytes per lane
    static constexpr int VB = EV * ES;
    static_assert(DK % G == 0 && DV % G == 0, "head dims split over G lanes");
    static_assert(KB % 4 == 0 && VB % 4 == 0, "lane slices are whole dwords");
};

template <int ES, int DK, int DV, int REP, int G, int NP, int NW>
struct AttnState {
    using C = AttnCfg<ES, DK, DV, REP, G, NP, NW>;
    float qr[REP][C::EK];
    float m[REP], l[REP];
    float acc[REP][C::EV];
};

// One wave step over positions blk0 + j*PW + grp, j < NP, of a page list.
// RT: the rows are a.pg.dk / a.pg.dv elements long (multiples of 4, at most
// DK / DV, the padded register layout); lanes load only their part of the
// true row, and the padding reads as zero.
template <bool MASK, bool RT, bool NT, int ES, int DK, int DV, int REP, int G, int NP, int NW>
__device__ __forceinline__ void attn_step(AttnState<ES, DK, DV, REP, G, NP, NW> &st,
                                          const AttnArgs &a, const int32_t *pages, uint32_t g,
                                          int blk0, int s0, int s1, int grp, int li)
{
    using C = AttnCfg<ES, DK, DV, REP, G, NP, NW>;
    const int P = 1 << a.pg.log2_page;
    const int dk = RT ? (int)a.pg.dk : DK, dv = RT ? (int)a.pg.dv : DV;
    Words<C::KB> kw[NP];
    Words<C::VB> vw[NP];
    float ks[NP], vs[NP];
    bool valid[NP];

#pragma unroll
    for (int j = 0; j < NP; j++) {
        const int blk = blk0 + j * C::PW;
        const int s = blk + grp;
        valid[j] = !MASK || (s >= s0 && s < s1);
        // The whole block of PW slots lies in one page (page_size % PW == 0)
        // and intersects [s0, s1), so its page is backed; an unbacked page
        // (never stored) reads as masked instead of faulting.
        const int32_t page = (!MASK || blk < s1) ? pages[blk >> a.pg.log2_page] : -1;
        if (page >= 0) {
            const uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
            // a masked lane reads the nearest slot in [s0, s1), inside the
            // same block, so that HBM serves only visible slots
            const int off = (MASK ? min(max(s, s0), s1 - 1) : s) & (P - 1);
            const uint8_t *kp = hb + (uint64_t)off * dk * ES + li * C::KB;
            const uint8_t *vp = hb + (uint64_t)P * dk * ES + (uint64_t)off * dv * ES + li * C::VB;
            if constexpr (RT) {
                load_words_upto<C::KB, NT>(kw[j], kp, dk * ES - li * C::KB);
                load_words_upto<C::VB, NT>(vw[j], vp, dv * ES - li * C::VB);
            } else {
                load_words<C::KB, NT>(kw[j], kp);
                load_words<C::VB, NT>(vw[j], vp);
            }
            if constexpr (ES == 1) {
                const float *sc = reinterpret_cast<const float *>(hb + (uint64_t)P * (dk + dv));
                ks[j] = sc[off];
                vs[j] = sc[P + off];
            } else {
                ks[j] = 1.0f;
                vs[j] = 1.0f;
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::KB / 4; i++)
                kw[j].w[i] = 0;
#pragma unroll
            for (int i = 0; i < C::VB / 4; i++)
                vw[j].w[i] = 0;
            ks[j] = 0.0f;
            vs[j] = 0.0f;
            valid[j] = false;
        }
        if constexpr (MASK && ES == 2) {
            // Unwritten slots may hold any bits (inf/nan in fp16): zero them.
#pragma unroll
            for (int i = 0; i < C::VB / 4; i++)
                vw[j].w[i] = valid[j] ? vw[j].w[i] : 0u;
        }
    }

    float vf[NP][C::EV];
#pragma unroll
    for (int j = 0; j < NP; j++)
#pragma unroll
        for (int e = 0; e < C::EV; e++)
            vf[j][e] = elem<ES>(vw[j].w, e);

#pragma unroll
    for (int t = 0; t < REP; t++) {
        float sc[NP];
#pragma unroll
        for (int j = 0; j < NP; j++) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < C::EK; e++)
                d = fmaf(st.qr[t][e], elem<ES>(kw[j].w, e), d);
            d = group_sum<G>(d);
            if constexpr (ES == 1)
                d *= ks[j];
            sc[j] = (MASK && !valid[j]) ? -INFINITY : d;
        }
        float mx = st.m[t];
#pragma unroll
        for (int j = 0; j < NP; j++)
            mx = fmaxf(mx, sc[j]);
        // Lazy running max: move it (and rescale the state) only when a score
        // exceeds it by more than 2^8, so the weights stay <= 256; otherwise
        // the rescale sweep over the accumulators is skipped for the whole
        // wave. The state (m, l, acc) is the same softmax up to rounding.
        const bool grow = mx > st.m[t] + 8.0f;
        if (__builtin_expect(__ballot(grow) != 0, 0)) {
            const float mnew = grow ? mx : st.m[t];
            const float r = fast_exp2(st.m[t] - mnew);
            st.m[t] = mnew;
            st.l[t] *= r;
#pragma unroll
            for (int e = 0; e < C::EV; e++)
                st.acc[t][e] *= r;
        }
        const float mref = st.m[t];
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const float p = fast_exp2(sc[j] - mref);
            st.l[t] += p;
            float pv = ES == 1 ? p * vs[j] : p;
            if constexpr (MASK)
                pv = valid[j] ? pv : 0.0f;
#pragma unroll
            for (int e = 0; e < C::EV; e++)
                st.acc[t][e] = fmaf(pv, vf[j][e], st.acc[t][e]);
        }
    }
}

template <bool RT, bool NT, int ES, int DK, int DV, int REP, int G, int NP, int NW>
__device__ __forceinline__ void attn_run(AttnState<ES, DK, DV, REP, G, NP, NW> &st, const AttnArgs &a,
                                         const int32_t *pages, uint32_t g, int s0, int s1, int wave,
                                         int grp, int li)
{
    using C = AttnCfg<ES, DK, DV, REP, G, NP, NW>;
    constexpr int BLK = C::PW * NP;
    const int start = (s0 / C::PW) * C::PW;
    for (int it = start + wave * BLK; it < s1; it += NW * BLK) {
        if (it >= s0 && it + BLK <= s1)
            attn_step<false, RT, NT>(st, a, pages, g, it, s0, s1, grp, li);
        else
            attn_step<true, RT, NT>(st, a, pages, g, it, s0, s1, grp, li);
    }
}

// Merge online-softmax state (m, l, acc) of another lane group / wave.
__device__ __forceinline__ void merge_state(float &m, float &l, float *acc, int n, float m2, float l2,
                                            const float *acc2)
{
    const float M = fmaxf(m, m2);
    const float ca = fast_exp2(m - M), cb = fast_exp2(m2 - M);
    l = l * ca + l2 * cb;
    for (int e = 0; e < n; e++)
        acc[e] = acc[e] * ca + acc2[e] * cb;
    m = M;
}

// A work-group is one (row, kv-head) unit, or with HS > 1 one of HS units
// that split the kv-head's query heads between them (REP each, REP * HS in
// the group): each reads the kv-head's K/V, so the per-lane state of a wide
// GQA group (heads x head dim) divides by HS and more units fit a CU.
// RT: head dims read at run time (a.pg.dk, a.pg.dv), DK / DV the padding.
template <int ES, int DK, int DV, int REP, int G, int NP, int NW, int HS, bool RT, bool PRE = false>
__global__ __launch_bounds__(64 * NW) void attend_kernel(AttnArgs a)
{
    using C = AttnCfg<ES, DK, DV, REP, G, NP, NW>;
    const int dk = RT ? (int)a.pg.dk : DK, dv = RT ? (int)a.pg.dv : DV;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane / G, li = lane % G;
    const uint32_t nkv = a.pg.nkv;
    // Work-group w runs on XCD w % 8. With 8-wave work-groups (long rows)
    // each XCD is given one contiguous run of units, so the work-groups
    // running on an XCD at one time read neighbouring rows (and their pages,
    // allocated in row order) rather than every eighth: the 4096-row decode
    // takes 0.748 ms per launch instead of 0.766. Short rows on 2-wave
    // work-groups keep the plain order: for them (the own positions of
    // sequences on a shared prefix) the runs measured no better, 0.0536 and
    // 0.0554 ms per layer step against 0.0521 and 0.0534. (The run is a
    // bijection on [0, gridDim.x): XCD x takes the gridDim.x / 8 units from
    // x * (gridDim.x / 8) + min(x, gridDim.x % 8), plus one when x <
    // gridDim.x % 8.)
    const uint32_t nwg = gridDim.x, xcd = blockIdx.x % 8u;
    const uint32_t unit = NW >= 8 ? (nwg / 8u) * xcd + min(xcd, nwg % 8u) + blockIdx.x / 8u : blockIdx.x;
    const uint32_t row = unit / (nkv * HS), gv = unit % (nkv * HS), g = gv / HS;   // heads gv*REP..+REP
    const uint32_t chunk = blockIdx.y + a.chunk_lo;

    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const SeqDev sd = a.seqs[seq];
    const int p = sd.pos + (a.row_t ? (int)a.row_t[row] : 0);
    const Visible vis = visible(sd, p, (int)a.pg.window);
    const int total = vis.n_sh + vis.n_own;
    const int nchunks = (total + (int)a.chunk - 1) / (int)a.chunk;
    if ((int)chunk >= nchunks)
        return;
    const int c0 = (int)chunk * (int)a.chunk, c1 = min(total, c0 + (int)a.chunk);

    // Fused KV append (decode step): the work-group whose chunk holds the new
    // position's slot stores it first (the engine stores before it attends,
    // engine/src/nd_model.c:2426-2454), then every wave reads it like any
    // other slot.
    if (HS == 1 && a.k_new) {      // (the host never fuses the store into a split launch)
        const int nslot = own_slot(sd, p, (int)a.pg.window);
        const int vi = vis.n_sh + nslot;
        if (vi >= c0 && vi < c1) {
            if (wave == 0) {
                const int32_t page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (nslot >> a.pg.log2_page)];
                if (page >= 0) {
                    const int P = 1 << a.pg.log2_page;
                    uint8_t *hb = const_cast<uint8_t *>(a.pool) + (uint64_t)page * a.pg.page_bytes +
                                  (uint64_t)g * a.pg.head_bytes;
                    const float kx = lane < dk ? a.k_new[((uint64_t)row * nkv + g) * dk + lane] : 0.0f;
                    const float vx = lane < dv ? a.v_new[((uint64_t)row * nkv + g) * dv + lane] : 0.0f;
                    store_row<ES>(hb, nslot & (P - 1), P, kx, vx, lane, dk, dv);
                }
            }
            // Workgroup-scope release/acquire + barrier: all waves of the group
            // share the CU's L1, so this is all the visibility the store needs
            // (an agent-scope fence would write back L2 from every group).
            __syncthreads();
        }
    }

    // A shared-prefix pass left chunk 0 (the prefix's softmax state) and this
    // is the row's only other chunk: the epilogue merges the two. In the
    // launches after such a pass (PRE), wave 0's first lane group requests
    // chunk 0 now, so that its latency overlaps the row's own loads rather
    // than ending the work-group (REP <= 2: its REP * (EV + 2) registers,
    // which other launches do not carry: held by the 4096-row decode's
    // kernel they cost it a wave per SIMD and 2-4%).
    constexpr bool PRE0 = PRE && REP <= 2;
    const bool merge0 = a.chunk_lo == 1 && nchunks == 2;
    float p0[PRE0 ? REP : 1][C::EV + 2] = {};
    if constexpr (PRE0) {
        if (merge0 && wave == 0 && lane < G) {
#pragma unroll
            for (int t = 0; t < REP; t++) {
                const float *r0 = a.part + ((uint64_t)row * a.nh + gv * REP + t) * a.max_chunks * (dv + 2);
#pragma unroll
                for (int e = 0; e < C::EV; e++)
                    p0[t][e] = (!RT || li * C::EV + e < dv) ? r0[li * C::EV + e] : 0.0f;
                p0[t][C::EV] = r0[dv];
                p0[t][C::EV + 1] = r0[dv + 1];
            }
        }
    }

    AttnState<ES, DK, DV, REP, G, NP, NW> st;
#pragma unroll
    for (int t = 0; t < REP; t++) {
        const float *qh = a.q + ((uint64_t)row * a.nh + gv * REP + t) * dk + li * C::EK;
#pragma unroll
        for (int e = 0; e < C::EK; e++)
            st.qr[t][e] = (!RT || li * C::EK + e < dk) ? qh[e] * a.qscale : 0.0f;
        st.m[t] = -FLT_MAX;
        st.l[t] = 0.0f;
#pragma unroll
        for (int e = 0; e < C::EV; e++)
            st.acc[t][e] = 0.0f;
    }

    if (c0 < vis.n_sh)
        attn_run<RT, false>(st, a, a.prefix_pages + (uint64_t)sd.prefix * a.pg.pages_per_seq, g, c0,
                     min(c1, vis.n_sh), wave, grp, li);
    if (c1 > vis.n_sh)
        attn_run<RT, true>(st, a, a.page_table + (uint64_t)seq * a.pg.pages_per_seq, g,
                     max(c0, vis.n_sh) - vis.n_sh, c1 - vis.n_sh, wave, grp, li);

    // Merge the lane groups of this wave: lanes li, li+G, li+2G, ...
#pragma unroll
    for (int t = 0; t < REP; t++) {
#pragma unroll
        for (int o = G; o < 64; o <<= 1) {
            float acc2[C::EV];
            const float m2 = __shfl_xor(st.m[t], o, 64);
            const float l2 = __shfl_xor(st.l[t], o, 64);
#pragma unroll
            for (int e = 0; e < C::EV; e++)
                acc2[e] = __shfl_xor(st.acc[t][e], o, 64);
            merge_state(st.m[t], st.l[t], st.acc[t], C::EV, m2, l2, acc2);
        }
    }

    // Merge the waves through LDS: [wave][t][li][EV + 2].
    constexpr int REC = C::EV + 2;
    __shared__ float lds[NW][REP][G][REC];
    if (NW > 1) {
        if (lane < G) {
#pragma unroll
            for (int t = 0; t < REP; t++) {
                float *r = lds[wave][t][li];
                r[0] = st.m[t];
                r[1] = st.l[t];
#pragma unroll
                for (int e = 0; e < C::EV; e++)
                    r[2 + e] = st.acc[t][e];
            }
        }
        __syncthreads();
        if (wave != 0)
            return;
        if (lane < G) {
#pragma unroll
            for (int w = 1; w < NW; w++)
#pragma unroll
                for (int t = 0; t < REP; t++) {
                    const float *r = lds[w][t][li];
                    merge_state(st.m[t], st.l[t], st.acc[t], C::EV, r[0], r[1], r + 2);
                }
        }
    }
    if (lane >= G)
        return;

#pragma unroll
    for (int t = 0; t < REP; t++) {
        const uint32_t h = gv * REP + t;
        if (nchunks == 1) {
            const float inv = 1.0f / st.l[t];
            float *o = a.out + ((uint64_t)row * a.nh + h) * dv + li * C::EV;
            const float *gt = a.gate ? a.gate + ((uint64_t)row * a.nh + h) * dv + li * C::EV : nullptr;
#pragma unroll
            for (int e = 0; e < C::EV; e++) {
                if (!RT || li * C::EV + e < dv) {
                    float z = st.acc[t][e] * inv;
                    if (gt)
                        z *= sigmoid_dev(gt[e]);
                    o[e] = z;
                }
            }
        } else if (merge0) {
            // merge chunk 0 (above) into this chunk and write the row
            const float *r0 = a.part + ((uint64_t)row * a.nh + h) * a.max_chunks * (dv + 2);
            const float m0 = PRE0 ? p0[PRE0 ? t : 0][C::EV] : r0[dv];
            const float l0 = PRE0 ? p0[PRE0 ? t : 0][C::EV + 1] : r0[dv + 1];
            const float M = fmaxf(st.m[t], m0);
            const float ca = fast_exp2(st.m[t] - M), cb = fast_exp2(m0 - M);
            const float inv = 1.0f / (st.l[t] * ca + l0 * cb);
            float *o = a.out + ((uint64_t)row * a.nh + h) * dv + li * C::EV;
            const float *gt = a.gate ? a.gate + ((uint64_t)row * a.nh + h) * dv + li * C::EV : nullptr;
#pragma unroll
            for (int e = 0; e < C::EV; e++) {
                if (!RT || li * C::EV + e < dv) {
                    const float a0 = PRE0 ? p0[PRE0 ? t : 0][e] : r0[li * C::EV + e];
                    float z = (st.acc[t][e] * ca + a0 * cb) * inv;
                    if (gt)
                        z *= sigmoid_dev(gt[e]);
                    o[e] = z;
                }
            }
        } else {
            float *r = a.part + (((uint64_t)row * a.nh + h) * a.max_chunks + chunk) * (dv + 2);
#pragma unroll
            for (int e = 0; e < C::EV; e++)
                if (!RT || li * C::EV + e < dv)
                    r[li * C::EV + e] = st.acc[t][e];
            if (li == 0) {
                r[dv] = st.m[t];
                r[dv + 1] = st.l[t];
            }
        }
    }
}

// Split-KV merge: one wave per (row, head), lane = output element (dv <= 64).
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs a)
{
    const int DV = (int)a.pg.dv;
    const int lane = threadIdx.x & 63;
    const uint64_t wid = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= (uint64_t)a.rows * a.nh)
        return;
    const uint32_t row = (uint32_t)(wid / a.nh), h = (uint32_t)(wid % a.nh);
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const SeqDev sd = a.seqs[seq];
    const int p = sd.pos + (a.row_t ? (int)a.row_t[row] : 0);
    const Visible vis = visible(sd, p, (int)a.pg.window);
    const int nchunks = (vis.n_sh + vis.n_own + (int)a.chunk - 1) / (int)a.chunk;
    if (nchunks <= 1 || (a.chunk_lo == 1 && nchunks == 2))    // (the attend kernel wrote the row)
        return;
    const float *base = a.part + ((uint64_t)row * a.nh + h) * a.max_chunks * (DV + 2);
    float M = -FLT_MAX;
    for (int c = 0; c < nchunks; c++)
        M = fmaxf(M, base[(uint64_t)c * (DV + 2) + DV]);
    float L = 0.0f, o = 0.0f;
    for (int c = 0; c < nchunks; c++) {
        const float *r = base + (uint64_t)c * (DV + 2);
        const float w = fast_exp2(r[DV] - M);
        L += r[DV + 1] * w;
        if (lane < DV)
            o += r[lane] * w;
    }
    if (lane < DV) {
        float z = o * (1.0f / L);
        if (a.gate)
            z *= sigmoid_dev(a.gate[((uint64_t)row * a.nh + h) * DV + lane]);
        a.out[((uint64_t)row * a.nh + h) * DV + lane] = z;
    }
}

// ------------------------------------------------------------- KV append

// One wave per (row, kv-head), lane = element (head dims <= 64).
template <int ES>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a)
{
    const int DK = (int)a.pg.dk, DV = (int)a.pg.dv;
    const int lane = threadIdx.x & 63;
    const uint64_t unit = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t nkv = a.pg.nkv;
    if (unit >= (uint64_t)a.rows * nkv)
        return;
    const uint32_t row = (uint32_t)(unit / nkv), g = (uint32_t)(unit % nkv);
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const SeqDev sd = a.seqs[seq];
    const int p = sd.pos + (a.row_t ? (int)a.row_t[row] : 0);
    const int slot = own_slot(sd, p, (int)a.pg.window);
    const int P = 1 << a.pg.log2_page;
    const int32_t page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (slot >> a.pg.log2_page)];
    if (page < 0)
        return;   // the host backs every appended slot; never taken
    uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
    const int off = slot & (P - 1);

    const float kx = lane < DK ? a.k[((uint64_t)row * nkv + g) * DK + lane] : 0.0f;
    const float vx = lane < DV ? a.v[((uint64_t)row * nkv + g) * DV + lane] : 0.0f;
    store_row<ES>(hb, off, P, kx, vx, lane, DK, DV);
}

// fp16 store with head dims that are multiples of 4: 16 lanes per (row,
// kv-head), four elements each (16-byte loads, 8-byte stores), four units
// per wave. Each unit is a short chain of dependent loads (sequence state,
// page id) before its store. A decode step's 4096 x 8 units run here as one
// wave per four units, one round on the chip, where one wave per unit took
// four rounds (13 us a launch). The row's K/V are loaded first: they do not
// depend on the page. The rounding is append_kernel's.
__global__ __launch_bounds__(256) void append_f16_kernel(AppendArgs a)
{
    const int DK = (int)a.pg.dk, DV = (int)a.pg.dv;
    const int e = 4 * (int)(threadIdx.x & 15);
    const uint64_t unit = (uint64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const uint32_t nkv = a.pg.nkv;
    if (unit >= (uint64_t)a.rows * nkv)
        return;
    const uint32_t row = (uint32_t)(unit / nkv), g = (uint32_t)(unit % nkv);
    float4 kx = {0.0f, 0.0f, 0.0f, 0.0f}, vx = kx;
    if (e < DK)
        kx = *reinterpret_cast<const float4 *>(a.k + ((uint64_t)row * nkv + g) * DK + e);
    if (e < DV)
        vx = *reinterpret_cast<const float4 *>(a.v + ((uint64_t)row * nkv + g) * DV + e);
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const SeqDev sd = a.seqs[seq];
    const int p = sd.pos + (a.row_t ? (int)a.row_t[row] : 0);
    const int slot = own_slot(sd, p, (int)a.pg.window);
    const int P = 1 << a.pg.log2_page;
    const int32_t page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (slot >> a.pg.log2_page)];
    if (page < 0)
        return;   // the host backs every appended slot; never taken
    uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
    const int off = slot & (P - 1);
    typedef _Float16 half4v __attribute__((ext_vector_type(4)));
    if (e < DK)
        *reinterpret_cast<half4v *>(hb + ((uint64_t)off * DK + e) * 2) =
            half4v{(_Float16)kx.x, (_Float16)kx.y, (_Float16)kx.z, (_Float16)kx.w};
    if (e < DV)
        *reinterpret_cast<half4v *>(hb + (uint64_t)P * DK * 2 + ((uint64_t)off * DV + e) * 2) =
            half4v{(_Float16)vx.x, (_Float16)vx.y, (_Float16)vx.z, (_Float16)vx.w};
}

// The int8 store in the same shape (16 lanes per unit, four elements each):
// the row's absmax over the 16 lanes by shuffles, then the engine's step
// sequence per element (quant_code), four codes stored as one word, the
// scales by the unit's first lane. Codes and scales are append_kernel<1>'s
// bit for bit: the max is exact in any order.
__global__ __launch_bounds__(256) void append_i8_kernel(AppendArgs a)
{
    const int DK = (int)a.pg.dk, DV = (int)a.pg.dv;
    const int e = 4 * (int)(threadIdx.x & 15);
    const uint64_t unit = (uint64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const uint32_t nkv = a.pg.nkv;
    if (unit >= (uint64_t)a.rows * nkv)
        return;       // (the 16 lanes of a unit leave together)
    const uint32_t row = (uint32_t)(unit / nkv), g = (uint32_t)(unit % nkv);
    float4 kx = {0.0f, 0.0f, 0.0f, 0.0f}, vx = kx;
    if (e < DK)
        kx = *reinterpret_cast<const float4 *>(a.k + ((uint64_t)row * nkv + g) * DK + e);
    if (e < DV)
        vx = *reinterpret_cast<const float4 *>(a.v + ((uint64_t)row * nkv + g) * DV + e);
    const uint32_t seq = a.row_seq ? a.row_seq[row] : row;
    const SeqDev sd = a.seqs[seq];
    const int p = sd.pos + (a.row_t ? (int)a.row_t[row] : 0);
    const int slot = own_slot(sd, p, (int)a.pg.window);
    const int P = 1 << a.pg.log2_page;
    const int32_t page = a.page_table[(uint64_t)seq * a.pg.pages_per_seq + (slot >> a.pg.log2_page)];
    float ak = fmaxf(fmaxf(fabsf(kx.x), fabsf(kx.y)), fmaxf(fabsf(kx.z), fabsf(kx.w)));
    float av = fmaxf(fmaxf(fabsf(vx.x), fabsf(vx.y)), fmaxf(fabsf(vx.z), fabsf(vx.w)));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
        ak = fmaxf(ak, __shfl_xor(ak, o, 16));
        av = fmaxf(av, __shfl_xor(av, o, 16));
    }
    if (page < 0)
        return;   // the host backs every appended slot; never taken
    uint8_t *hb = a.pool + (uint64_t)page * a.pg.page_bytes + (uint64_t)g * a.pg.head_bytes;
    const int off = slot & (P - 1);
    const float sk = ak > 0.0f ? __fdiv_rn(ak, 127.0f) : 1.0f;
    const float sv = av > 0.0f ? __fdiv_rn(av, 127.0f) : 1.0f;
    const float rk = __fdiv_rn(1.0f, sk), rv = __fdiv_rn(1.0f, sv);
    auto pack = [](float x0, float x1, float x2, float x3, float s_, float r_) {
        return (uint32_t)(uint8_t)quant_code(x0, s_, r_) | (uint32_t)(uint8_t)quant_code(x1, s_, r_) << 8 |
               (uint32_t)(uint8_t)quant_code(x2, s_, r_) << 16 | (uint32_t)(uint8_t)quant_code(x3, s_, r_) << 24;
    };
    if (e < DK)
        *reinterpret_cast<uint32_t *>(hb + (uint64_t)off * DK + e) = pack(kx.x, kx.y, kx.z, kx.w, sk, rk);
    if (e < DV)
        *reinterpret_cast<uint32_t *>(hb + (uint64_t)P * DK + (uint64_t)off * DV + e) =
            pack(vx.x, vx.y, vx.z, vx.w, sv, rv);
    if (e == 0) {
        float *sc = reinterpret_cast<float *>(hb + (uint64_t)P * (DK + DV));
        sc[off] = sk;
        sc[P + off] = sv;
    }
}

// ------------------------------------------------------ copies and staging

// Bytes of one slot of one kv-head: K row, V row (+ the two scales).
template <int ES>
__device__ __forceinline__ void copy_slot(uint8_t *dhb, int doff, const uint8_t *shb, int soff, int P,
                                          int tid, int nthr, int DK, int DV)
{
    const uint32_t *sk = reinterpret_cast<const uint32_t *>(shb + (uint64_t)soff * DK * ES);
    uint32_t *dk = reinterpret_cast<uint32_t *>(dhb + (uint64_t)doff * DK * ES);
    for (int i = tid; i < DK * ES / 4; i += nthr)
        dk[i] = sk[i];
    const uint32_t *sv = reinterpret_cast<const uint32_t *>(shb + (uint64_t)P * DK * ES + (uint64_t)soff * DV * ES);
    uint32_t *dv = reinterpret_cast<uint32_t *>(dhb + (uint64_t)P * DK * ES + (uint64_t)doff * DV * ES);
    for (int i = tid; i < DV * ES / 4; i += nthr)
        dv[i] = sv[i];
    if (ES == 1 && tid == 0) {
        const float *ss = reinterpret_cast<const float *>(shb + (uint64_t)P * (DK + DV));
        float *ds = reinterpret_cast<float *>(dhb + (uint64_t)P * (DK + DV));
        ds[doff] = ss[soff];
        ds[P + doff] = ss[P + soff];
    }
}

// grid (count, n_layers), one block per (slot, layer), heads in a loop.
template <int ES>
__global__ __launch_bounds__(64) void copy_kernel(CopyArgs a)
{
    const uint32_t i = blockIdx.x, l = blockIdx.y;
    if (i >= a.count || l >= a.n_layers)
        return;
    const int P = 1 << a.pg.log2_page;
    const uint32_t ss = a.src_slot0 + i, ds = a.dst_slot0 + i;
    const int32_t spg = a.src_pages[ss >> a.pg.log2_page], dpg = a.dst_pages[ds >> a.pg.log2_page];
    if (spg < 0 || dpg < 0)
        return;
    const uint8_t *sp = a.pool + l * a.pg.layer_bytes + (uint64_t)spg * a.pg.page_bytes;
    uint8_t *dp = a.pool + l * a.pg.layer_bytes + (uint64_t)dpg * a.pg.page_bytes;
    for (uint32_t g = 0; g < a.pg.nkv; g++)
        copy_slot<ES>(dp + g * a.pg.head_bytes, ds & (P - 1), sp + g * a.pg.head_bytes, ss & (P - 1), P,
                      threadIdx.x, blockDim.x, (int)a.pg.dk, (int)a.pg.dv);
}

// One block per staged position: pool <-> [count][nkv][d] staging.
template <int ES, bool SCATTER>
__global__ __launch_bounds__(64) void stage_kernel(StageArgs a)
{
    const int DK = (int)a.pg.dk, DV = (int)a.pg.dv;
    const uint32_t i = blockIdx.x;
    if (i >= a.count)
        return;
    const int P = 1 << a.pg.log2_page;
    const int off = (int)a.slot_in_page[i];
    uint8_t *pp = a.pool + (uint64_t)a.pages_for_slot[i] * a.pg.page_bytes;
    for (uint32_t g = 0; g < a.pg.nkv; g++) {
        uint8_t *hb = pp + g * a.pg.head_bytes;
        uint8_t *kr = hb + (uint64_t)off * DK * ES;
        uint8_t *vr = hb + (uint64_t)P * DK * ES + (uint64_t)off * DV * ES;
        uint8_t *sk = a.stage_k + ((uint64_t)i * a.pg.nkv + g) * DK * ES;
        uint8_t *sv = a.stage_v + ((uint64_t)i * a.pg.nkv + g) * DV * ES;
        for (int b = threadIdx.x; b < DK * ES; b += blockDim.x) {
            if (SCATTER)
                kr[b] = sk[b];
            else
                sk[b] = kr[b];
        }
        for (int b = threadIdx.x; b < DV * ES; b += blockDim.x) {
            if (SCATTER)
                vr[b] = sv[b];
            else
                sv[b] = vr[b];
        }
        if (threadIdx.x == 0) {
            float *sc = reinterpret_cast<float *>(hb + (uint64_t)P * (DK + DV));
            float *dks = a.stage_ks + (uint64_t)i * a.pg.nkv + g;
            float *dvs = a.stage_vs + (uint64_t)i * a.pg.nkv + g;
            if (ES == 1) {
                if (SCATTER) {
                    sc[off] = *dks;
                    sc[P + off] = *dvs;
                } else {
                    *dks = sc[off];
                    *dvs = sc[P + off];
                }
            } else if (!SCATTER) {
                *dks = 1.0f;
                *dvs = 1.0f;
            }
        }
    }
}

// pos += n for the listed sequences (the engine's pos++, nd_model.c:3094).
__global__ __launch_bounds__(256) void advance_kernel(SeqDev *seqs, const uint32_t *seq_list, uint32_t nseq,
                                                      uint32_t n)
{
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < nseq)
        seqs[seq_list ? seq_list[b] : b].pos += (int32_t)n;
}

// --------------------------------------------------------- synthetic data

__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// N(0,1) from one 64-bit hash: Box-Muller on two 24-bit uniforms.
__device__ __forceinline__ float normal_from(uint64_t h)
{
    const float u1 = ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = (float)(uint32_t)(h & 0xFFFFFFu) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * __logf(u1)) * __cosf(6.28318530717958647f * u2);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(void *dst, uint64_t n, int dtype, uint64_t seed,
                                                          float scale)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float x = normal_from(splitmix64(seed ^ splitmix64(i))) * scale;
        if (dtype == 0)
            static_cast<float *>(dst)[i] = x;
        else
            static_cast<_Float16 *>(dst)[i] = (_Float16)x;
    }
}

// Fill own slots [0, n_own) of every listed sequence. The value of
// (layer, seq, slot, head, element) depends on those indices only. ES 1:
// int8 codes round(32 x) clamped to +-127 with scales 1/32, so the
// dequantised values are N(0,1) to within the code step.
template <int ES>
__global__ __launch_bounds__(256) void fill_kv_kernel(FillKvArgs a)
{
    const uint32_t DK = a.pg.dk, DV = a.pg.dv;
    const uint32_t bi = blockIdx.x, l = blockIdx.y;
    if (bi >= a.nseq || l >= a.n_layers)
        return;
    const uint32_t seq = a.seq_list ? a.seq_list[bi] : bi;
    const SeqDev sd = a.seqs[seq];
    if (sd.pos <= 0)
        return;
    const Visible vis = visible(sd, sd.pos - 1, (int)a.pg.window);
    const int P = 1 << a.pg.log2_page;
    const uint32_t nkv = a.pg.nkv;
    const uint64_t per_slot = (uint64_t)nkv * (DK + DV);
    const uint64_t total = (uint64_t)vis.n_own * per_slot;
    const uint64_t key = a.seed ^ splitmix64(((uint64_t)l << 40) ^ ((uint64_t)seq << 8) ^ 0x5a5aull);
    uint8_t *lp = a.pool + l * a.pg.layer_bytes;
    const int32_t *pages = a.page_table + (uint64_t)seq * a.pg.pages_per_seq;
    for (uint64_t i = threadIdx.x; i < total; i += blockDim.x) {
        const uint32_t slot = (uint32_t)(i / per_slot);
        const uint32_t rem = (uint32_t)(i % per_slot);
        const uint32_t g = rem / (DK + DV), e = rem % (DK + DV);
        const int32_t pg = pages[slot >> a.pg.log2_page];
        if (pg < 0)
            continue;
        uint8_t *hb = lp + (uint64_t)pg * a.pg.page_bytes + g * a.pg.head_bytes;
        const int off = slot & (P - 1);
        const float z = normal_from(splitmix64(key + i));
        if constexpr (ES == 2) {
            const _Float16 x = (_Float16)z;
            if (e < DK)
                reinterpret_cast<_Float16 *>(hb + (uint64_t)off * DK * 2)[e] = x;
            else
                reinterpret_cast<_Float16 *>(hb + (uint64_t)P * DK * 2 + (uint64_t)off * DV * 2)[e - DK] = x;
        } else {
            const int8_t c = (int8_t)(int)fminf(fmaxf(__builtin_rintf(z * 32.0f), -127.0f), 127.0f);
            if (e < DK)
                reinterpret_cast<int8_t *>(hb + (uint64_t)off * DK)[e] = c;
            else
                reinterpret_cast<int8_t *>(hb + (uint64_t)P * DK + (uint64_t)off * DV)[e - DK] = c;
            float *sc = reinterpret_cast<float *>(hb + (uint64_t)P * (DK + DV));
            if (e == 0)
                sc[off] = 1.0f / 32.0f;
            else if (e == DK)
                sc[P + off] = 1.0f / 32.0f;
        }
    }
}

// ------------------------------------------------------------- dispatch

// Lanes per KV position: 16-byte row slices (8 fp16 or 16 int8 elements);
// 8-byte int8 slices for the widest GQA group, whose per-lane state would
// not fit in registers otherwise.
template <int ES, int DK, int REP>
constexpr int lanes_per_pos() { return ES == 2 ? 8 : ((REP >= 8 && DK % 64 == 0) ? 8 : 4); }

// Waves per decode work-group. Wide GQA (rep >= 4): one, since each lane
// carries rep heads of state and the cross-wave merge would cost more than
// it parallelises (rows of a few hundred positions: 4.4x faster at 12 q /
// 2 kv heads, int8). MHA and narrow GQA: eight for work items of 448
// positions or more, whose rows split across many waves; two below, where
// 8-wave groups leave the chip with too few of them (1024 sequences on a
// 213-token prefix, ~300 positions: 1.59 M against 1.21 M tokens/s; 4096
// rows of 213-1024: eight is 6% faster). NDA_ATT_NW fixes one value for
// every geometry (a build-time tuning knob).
template <int REP>
constexpr int att_nw(bool long_items)
{
#ifdef NDA_ATT_NW
    return NDA_ATT_NW;
#else
    return REP >= 4 ? 1 : (long_items ? 8 : 2);
#endif
}
constexpr uint32_t ATT_LONG_ITEM = 448;

// Positions per lane group per step. fp16 at rep <= 2: 4 (80 registers, 6
// waves per SIMD); 8 also fits without spilling (120 registers) but leaves 4
// waves per SIMD, and the 4096-row decode then ran 14% slower (7.33 against
// 6.30 ms per step): waves in flight count for more than loads per wave. The
// int8 and wide-GQA states are larger.
template <int ES, int REP>
constexpr int att_np()
{
#ifdef NDA_ATT_NP
    return NDA_ATT_NP;
#else
    return (ES == 2 && REP <= 2) ? 4 : (REP <= 2 ? 2 : 1);
#endif
}

static inline int es_of(const Geo &g) { return g.kv_f16 ? 2 : 1; }

bool geometry_fast(const Geo &g)
{
#define X(ES, DK, DV, REP) if (es_of(g) == ES && g.dk == DK && g.dv == DV && g.rep == REP) return true;
    NDA_FOR_GEOMETRIES(X)
#undef X
    return false;
}

// The shapes the engine's attn_heads defines (engine/include/nd_model.h:244-245,
// engine/src/nd_model.c:2118-2139): head dims up to ND_KV_HD_CAP (64) and up
// to ND_KV_REP_CAP (8) query heads per kv-head. Its staging converts whole
// 4-byte words of codes (kv_stage_pair, :79-94) and its P.V loops step four
// elements, so only head dims that are multiples of 4 are well defined there.
bool geometry_supported(const Geo &g)
{
    return g.dk >= 4 && g.dk <= 64 && g.dk % 4 == 0 && g.dv >= 4 && g.dv <= 64 && g.dv % 4 == 0 &&
           g.rep >= 1 && g.rep <= 8;
}

static inline unsigned blocks_for(uint64_t waves) { return (unsigned)((waves + 3) / 4); }

// Query heads per work-group for a GQA group of REP: the widest even groups
// (rep 6, 8) split in two, except when the launch also stores the new row
// (one work-group per kv-head must own that store).
template <int REP>
constexpr int att_hs()
{
#ifdef NDA_ATT_HS
    return REP % NDA_ATT_HS == 0 ? NDA_ATT_HS : 1;
#else
    return REP >= 6 && REP % 2 == 0 ? 2 : 1;
#endif
}

// Lanes per position of the padded (run-time dims) instances: 8, so a lane
// holds 8 elements of K and of V (16-byte fp16 or 8-byte int8 slices).
template <int ES, int REP>
constexpr int lanes_rt() { return 8; }

template <int ES, int DK, int DV, int REP, int HS, int NW, bool RT, bool PRE = false>
static void launch_attend_hs(const AttnArgs &a, hipStream_t s)
{
    constexpr int R = REP / HS;
    constexpr int G = RT ? lanes_rt<ES, R>() : lanes_per_pos<ES, DK, R>();
    const dim3 grid(a.rows * a.pg.nkv * HS, a.max_chunks - a.chunk_lo);
    hipLaunchKernelGGL((attend_kernel<ES, DK, DV, R, G, att_np<ES, R>(), NW, HS, RT, PRE>), grid, dim3(64 * NW), 0,
                       s, a);
}

template <int ES, int DK, int DV, int REP, bool RT>
static void launch_attend_geo(const AttnArgs &a, bool long_items, hipStream_t s)
{
    if (att_hs<REP>() > 1 && !a.k_new)
        launch_attend_hs<ES, DK, DV, REP, att_hs<REP>(), 1, RT>(a, s);
    else if (long_items)
        launch_attend_hs<ES, DK, DV, REP, 1, att_nw<REP>(true), RT>(a, s);
    else {
        if constexpr (REP <= 2) {
            if (a.chunk_lo == 1) {      // after a shared-prefix pass: chunk 0 requested early
                launch_attend_hs<ES, DK, DV, REP, 1, att_nw<REP>(false), RT, true>(a, s);
                return;
            }
        }
        launch_attend_hs<ES, DK, DV, REP, 1, att_nw<REP>(false), RT>(a, s);
    }
}

// Shapes outside NDA_FOR_GEOMETRIES: dims padded to 64, one instance per
// (element size, rep).
#define NDA_RT_REPS(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)

hipError_t launch_attend(const Geo &g, const AttnArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    if (!geometry_supported(g) || (int)a.pg.dk != g.dk || (int)a.pg.dv != g.dv)
        return hipErrorNotSupported;
    const bool long_items = (a.avg_len < a.chunk ? a.avg_len : a.chunk) >= ATT_LONG_ITEM;
#define X(ES, DK, DV, REP)                                                                      \
    if (es_of(g) == ES && g.dk == DK && g.dv == DV && g.rep == REP) {                          \
        launch_attend_geo<ES, DK, DV, REP, false>(a, long_items, s);                            \
        return hipGetLastError();                                                               \
    }
    NDA_FOR_GEOMETRIES(X)
#undef X
#define X(REP)                                                                                  \
    if (g.rep == REP) {                                                                         \
        if (g.kv_f16)                                                                           \
            launch_attend_geo<2, 64, 64, REP, true>(a, long_items, s);                          \
        else                                                                                    \
            launch_attend_geo<1, 64, 64, REP, true>(a, long_items, s);                          \
        return hipGetLastError();                                                               \
    }
    NDA_RT_REPS(X)
#undef X
    return hipErrorNotSupported;
}

hipError_t launch_combine(const Geo &g, const AttnArgs &a, hipStream_t s)
{
    // after a shared-prefix pass, rows of two chunks are merged by the attend
    // kernel itself
    if (a.rows == 0 || a.max_chunks <= 1 || (a.chunk_lo == 1 && a.max_chunks == 2))
        return hipSuccess;
    if (g.dv > 64)
        return hipErrorNotSupported;
    hipLaunchKernelGGL(combine_kernel, dim3(blocks_for((uint64_t)a.rows * a.nh)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_append(const Geo &g, const AppendArgs &a, hipStream_t s)
{
    if (a.rows == 0)
        return hipSuccess;
    if (!geometry_supported(g))
        return hipErrorNotSupported;
    const uint64_t units = (uint64_t)a.rows * a.pg.nkv;
    const unsigned nb = blocks_for(units);
    const bool vec = g.dk % 4 == 0 && g.dv % 4 == 0 && (reinterpret_cast<uintptr_t>(a.k) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.v) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL((g.kv_f16 ? append_f16_kernel : append_i8_kernel), dim3((unsigned)((units + 15) / 16)),
                           dim3(256), 0, s, a);
    else if (g.kv_f16)
        hipLaunchKernelGGL((append_kernel<2>), dim3(nb), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((append_kernel<1>), dim3(nb), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_copy(const Geo &g, const CopyArgs &a, hipStream_t s)
{
    if (a.count == 0 || a.n_layers == 0)
        return hipSuccess;
    if (g.kv_f16)
        hipLaunchKernelGGL((copy_kernel<2>), dim3(a.count, a.n_layers), dim3(64), 0, s, a);
    else
        hipLaunchKernelGGL((copy_kernel<1>), dim3(a.count, a.n_layers), dim3(64), 0, s, a);
    return hipGetLastError();
}

static hipError_t launch_stage(const Geo &g, const StageArgs &a, hipStream_t s, bool scatter)
{
    if (a.count == 0)
        return hipSuccess;
    if (g.kv_f16) {
        if (scatter)
            hipLaunchKernelGGL((stage_kernel<2, true>), dim3(a.count), dim3(64), 0, s, a);
        else
            hipLaunchKernelGGL((stage_kernel<2, false>), dim3(a.count), dim3(64), 0, s, a);
    } else {
        if (scatter)
            hipLaunchKernelGGL((stage_kernel<1, true>), dim3(a.count), dim3(64), 0, s, a);
        else
            hipLaunchKernelGGL((stage_kernel<1, false>), dim3(a.count), dim3(64), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_gather(const Geo &g, const StageArgs &a, hipStream_t s) { return launch_stage(g, a, s, false); }
hipError_t launch_scatter(const Geo &g, const StageArgs &a, hipStream_t s) { return launch_stage(g, a, s, true); }

hipError_t launch_fill_kv(const Geo &g, const FillKvArgs &a, hipStream_t s)
{
    if (a.nseq == 0 || a.n_layers == 0)
        return hipSuccess;
    dim3 grid(a.nseq, a.n_layers);
    if (g.kv_f16)
        hipLaunchKernelGGL((fill_kv_kernel<2>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((fill_kv_kernel<1>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_advance(SeqDev *seqs, const uint32_t *seq_list, uint32_t nseq, uint32_t n, hipStream_t s)
{
    if (nseq == 0)
        return hipSuccess;
    hipLaunchKernelGGL(advance_kernel, dim3((nseq + 255) / 256), dim3(256), 0, s, seqs, seq_list, nseq, n);
    return hipGetLastError();
}

hipError_t launch_fill_normal(void *dst, uint64_t n, int dtype, uint64_t seed, float scale, hipStream_t s)
{
    if (n == 0)
        return hipSuccess;
    uint64_t nb = (n + 255) / 256;
    if (nb > 65536)
        nb = 65536;
    hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)nb), dim3(256), 0, s, dst, n, dtype, seed, scale);
    return hipGetLastError();
}

} // namespace nda
