// nda_ctx.h - the context behind the C ABI of libndattn (include/nda.h) and
// the host helpers its translation units share:
//   nda_api_ctx.hip      context lifecycle, buffers and uploads, sequence and
//                        prefix state, KV inspection, memory and device calls
//   nda_api_decode.hip   KV append, decode (split-KV, shared-prefix pass,
//                        GQA on MFMA), nda_step, nda_decode_noalloc
//   nda_api_prefill.hip  causal prefill planning and launch
//   nda_api_front.hip    the attention front (taps, norms, rotary) and
//                        nda_attention
//   nda_api_cq.hip       CQ tensors and the attention block calls
//
// The host keeps the authoritative copy of every sequence's state (pos,
// n_sink, attached prefix) and of the page tables, the way the engine keeps
// them in nd_model (engine/include/nd_model.h:132-148); the device copies are
// refreshed on the caller's stream right before the launch that reads them.
#ifndef NDA_CTX_H
#define NDA_CTX_H

#include "nda.h"
#include "nda_internal.h"
#include "nda_state.h"

#include <algorithm>
#include <array>
#include <cstdint>
#include <string>
#include <vector>

using namespace nda;
using namespace nda_host;

namespace nda_host {

struct ProfRec {
    int kind;
    hipEvent_t a, b;
};

// An upload in flight from the pinned ring: bytes [lo, hi) of the ring, free
// again once `ev` (recorded behind the copy) has completed.
struct UploadRec {
    size_t lo, hi;
    hipEvent_t ev;
};

constexpr size_t UPLOAD_RING_BYTES = 16u << 20;
constexpr int UPLOAD_EVENTS = 256;

} // namespace nda_host

struct nda_ctx {
    nda_config cfg{};
    Geo geo{};
    PageGeom pg{};
    uint64_t max_pages = 0;
    uint32_t chunk = 0;                 // fixed split size, 0 = chosen per launch
    int cus = 256;

    uint8_t *pool = nullptr;            // n_layers * layer_bytes
    int32_t *d_pages = nullptr;         // [max_seqs][pps]
    int32_t *d_prefix_pages = nullptr;  // [max_prefixes][pps]
    SeqDev *d_seqs = nullptr;
    uint32_t *d_rows = nullptr;         // row_seq | row_t staging
    size_t rows_cap = 0;
    float *d_part = nullptr;
    size_t part_cap = 0;                // floats
    uint8_t *d_stage = nullptr;
    size_t stage_cap = 0;
    uint32_t *d_pf = nullptr;           // prefill work list staging
    size_t pf_cap = 0;                  // uint32 entries
    // GQA decode work order (longest rows first) for batches of sequences
    // 0..rows-1, valid while no sequence state has changed since it was built
    uint32_t *d_order = nullptr;
    size_t order_cap = 0;               // uint32 entries
    uint32_t order_rows = 0;
    uint64_t order_ver = 0;
    uint64_t state_ver = 1;             // bumped by every change of a sequence's position, sinks or prefix
    uint64_t dev_bytes = 0;
    uint8_t *scratch = nullptr;         // this device's nda_decode_noalloc scratch

    PageTables pt;                      // page tables, free list, journal (host mirror)
    std::vector<SeqHost> seqs;
    std::vector<Prefix> prefixes;
    bool seqs_dirty = true;

    // attention front (nda_front_init): tap histories, weights, rotary table
    uint32_t taps = 0, max_pos = 0, dcol = 0;
    uint64_t hist_block = 0;            // floats per sequence: n_layers * taps * dcol
    float *d_hist = nullptr;            // [max_seqs] blocks, live
    float *d_snap_hist = nullptr;       // [max_seqs] blocks, restored by rewind
    float *d_prefix_hist = nullptr;     // [max_prefixes] blocks
    float *d_front_w = nullptr;         // [n_layers][taps][dcol]
    float *d_front_norm = nullptr;      // [n_layers][2][qk]
    float2 *d_rope = nullptr;           // [max_pos][qk/2]
    std::vector<uint8_t> front_w_set;   // per layer
    float *d_qfront = nullptr;          // nda_attention's normalised q
    size_t qfront_cap = 0;              // floats
    uint32_t *d_front_rows = nullptr;   // row_seq | row_t | row_n
    size_t front_rows_cap = 0;          // uint32 entries
    HistOp *d_hist_ops = nullptr;
    size_t hist_ops_cap = 0;
    std::vector<HistOp> hist_pending;   // applied in order before the next front launch
    std::vector<uint8_t> seen;          // duplicate-id scratch

    // attention block (nda_block_weights): per layer q, k, v, gate, out_proj
    std::vector<std::array<const nda_cq *, 5>> blk;
    uint32_t d_model = 0;
    float *d_bscr = nullptr;            // xh | q | k | v | gate | attn | attn xh, per row
    size_t bscr_cap = 0;                // floats

    // pinned staging of the per-call uploads (upload()); null: none could be
    // allocated, uploads copy from pageable memory
    uint8_t *h_ring = nullptr;
    size_t ring_cap = 0, ring_head = 0;
    UploadRec ring_live[UPLOAD_EVENTS]; // in flight, in ring order: a circular list
    int live_head = 0, live_n = 0;
    std::vector<hipEvent_t> ring_ev;    // free events, all created with the context (capacity reserved)

    // stream order: the stream of the last call that queued work, and the
    // event a call on another stream waits for (on_stream)
    hipStream_t last_stream = nullptr;
    bool has_stream = false;
    hipEvent_t order_ev = nullptr;

    bool prof = false;
    std::vector<ProfRec> prof_pending;
    std::vector<hipEvent_t> ev_free;
    double prof_ms[NDA_K_COUNT] = {};
    uint64_t prof_n[NDA_K_COUNT] = {};

    std::string err;
};

namespace nda_host {

// ---- allocation (the engine's ND_ALLOC / ND_FREE seam, nda_set_allocator)

void *dev_alloc(size_t bytes);
void dev_free(void *p);
// This device's address of nda_decode_noalloc's scratch array.
hipError_t scratch_address(int dev, uint8_t **out);

// ---- errors

int fail(nda_ctx *c, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int hip_fail(nda_ctx *c, hipError_t e, const char *what);

#define HIPC(c, call)                                      \
    do {                                                   \
        hipError_t e_ = (call);                            \
        if (e_ != hipSuccess)                              \
            return hip_fail((c), e_, #call);               \
    } while (0)

// ---- stream order, uploads, pages

int on_stream(nda_ctx *c, hipStream_t st);
int upload(nda_ctx *c, void *dst, const void *src, size_t n, hipStream_t st);
void release_pages(nda_ctx *c, uint32_t seq);
int back_slots(nda_ctx *c, uint32_t seq, uint32_t s0, uint32_t s1);
int back_positions(nda_ctx *c, uint32_t seq, uint32_t p0, uint32_t n);
int sync_tables(nda_ctx *c, hipStream_t st);

// ---- device staging buffers

// Grows a device staging buffer to n_alloc elements of T when it holds fewer
// than `need`. The new buffer is allocated first: a failed allocation returns
// NDA_ERR_NOMEM with the old buffer and the context unchanged. Queued
// launches may still read the old buffer, so the device is drained before it
// is freed.
template <typename T>
int grow_buf(nda_ctx *c, T *&buf, size_t &cap, size_t need, size_t n_alloc)
{
    if (need <= cap)
        return NDA_OK;
    T *nb = static_cast<T *>(dev_alloc(n_alloc * sizeof(T)));
    if (!nb)
        return fail(c, NDA_ERR_NOMEM, "device allocation of %zu bytes failed", n_alloc * sizeof(T));
    if (buf) {
        if (hipError_t e = hipDeviceSynchronize(); e != hipSuccess) {
            dev_free(nb);
            return hip_fail(c, e, "hipDeviceSynchronize (buffer growth)");
        }
        dev_free(buf);
        c->dev_bytes -= cap * sizeof(T);
    }
    buf = nb;
    cap = n_alloc;
    c->dev_bytes += n_alloc * sizeof(T);
    return NDA_OK;
}

int ensure_rows(nda_ctx *c, size_t rows);
int ensure_part(nda_ctx *c, size_t floats);
int ensure_pf(nda_ctx *c, size_t n);
int ensure_stage(nda_ctx *c, size_t bytes);

template <typename T>
int ensure_buf(nda_ctx *c, T *&buf, size_t &cap, size_t need)
{
    return grow_buf(c, buf, cap, need, std::max<size_t>(need, 4096));
}

// ---- profiling events

hipEvent_t take_event(nda_ctx *c);

struct ProfScope {
    nda_ctx *c;
    int kind;
    hipStream_t st;
    hipEvent_t a = nullptr, b = nullptr;
    ProfScope(nda_ctx *c_, int k, hipStream_t s, bool on = true) : c(c_), kind(k), st(s)
    {
        if (c->prof && on) {
            a = take_event(c);
            b = take_event(c);
            if (a && b)
                (void)hipEventRecord(a, st);
        }
    }
    ~ProfScope()
    {
        if (a && b) {
            (void)hipEventRecord(b, st);
            c->prof_pending.push_back({kind, a, b});
        } else {
            if (a)
                c->ev_free.push_back(a);
            if (b)
                c->ev_free.push_back(b);
        }
    }
};

// ---- argument checks

int check_seq(nda_ctx *c, uint32_t seq);
int check_ids(nda_ctx *c, uint32_t nseq, const uint32_t *ids);

inline uint32_t sid(const uint32_t *ids, uint32_t b) { return ids ? ids[b] : b; }

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// ---- tap histories of the attention front

float *hist_live(nda_ctx *c, uint32_t seq);
float *hist_snap(nda_ctx *c, uint32_t seq);
float *hist_prefix(nda_ctx *c, int32_t id);
// Queue a whole-block copy (src null: clear). Calls without a stream
// (reset, rewind) only queue; the queue is applied in order on the caller's
// stream before the next front launch or history read.
void hist_queue(nda_ctx *c, float *dst, const float *src);
int hist_flush(nda_ctx *c, hipStream_t st);
int hist_reserve(nda_ctx *c, size_t extra);

// ---- attention launches

int upload_rows(nda_ctx *c, uint32_t rows, const uint32_t *row_seq, const uint32_t *row_t,
                hipStream_t st, const uint32_t **d_seq, const uint32_t **d_t);
uint32_t pick_chunk(const nda_ctx *c, uint64_t units, uint64_t sum_total, uint32_t max_total);
AttnArgs attn_args(nda_ctx *c, uint32_t layer, uint32_t rows, const float *q, const float *gate,
                   float *out, uint32_t max_total, uint64_t sum_total);
bool mfma_decode_geo(const nda_ctx *c);
bool mfma_decode(const nda_ctx *c, const AttnArgs &a);
int reserve_attend(nda_ctx *c, uint32_t rows, bool staged, uint32_t max_total, uint64_t sum_total);
// part: split-KV partials of at least rows * nh * max_chunks * (v_hd + 2)
// floats, or null for the context's own buffer (grown on demand). prof: record
// profiling events (nda_decode_noalloc records none: creating an event may
// allocate). ordered: the GQA decode may take the rows longest first (it then
// builds or reuses the context's order buffer; nda_decode_noalloc does not).
int run_attend(nda_ctx *c, AttnArgs &a, hipStream_t st, float *part = nullptr, bool prof = true,
               bool ordered = true);

// ---- shared between the ABI groups

// decode (nda_api_decode.hip): the store (k, v non-null) and attention of one
// token per listed sequence, as nda_step without the front
int decode_impl(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
                const float *k, const float *v, const float *gate, float *out, void *stream);

// prefill (nda_api_prefill.hip)
// What one nda_prefill call launches: rows, the visible runs they attend,
// the kernel (VALU or MFMA) and the MFMA work-group size and work list.
struct PrefillPlan {
    uint64_t rows = 0, sum_total = 0;
    uint32_t max_total = 0, rep = 1, trows = 0, nseq = 0;
    int waves = 4;
    bool valu = false;
    size_t n_items = 0;
};
int prefill_check(nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens);
int prefill_plan(nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens, PrefillPlan &pl);
int prefill_reserve(nda_ctx *c, const PrefillPlan &pl);

// the front (nda_api_front.hip): initialised, weights present, each
// sequence at most once, every position inside the rotary table
int front_check(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens);

} // namespace nda_host

#endif
