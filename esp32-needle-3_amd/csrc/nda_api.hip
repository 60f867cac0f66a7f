// nda_api.hip - the C ABI of libndattn (include/nda.h): context, paged KV
// pool, per-sequence session state, shared prefix segments and launches.
//
// The host keeps the authoritative copy of every sequence's state (pos,
// n_sink, attached prefix) and of the page tables, the way the engine keeps
// them in nd_model (engine/include/nd_model.h:132-148); the device copies are
// refreshed on the caller's stream right before the launch that reads them.
#include "nda.h"
#include "nda_internal.h"
#include "nda_state.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_set>
#include <vector>

using namespace nda;
using namespace nda_host;

// Scratch of nda_decode_noalloc: the launch's sequence ids, then its split-KV
// partials. One array per GPU, held until the process ends. Host code never
// uses this name as an address (on the host it is only a stand-in): each
// device's address comes from hipGetSymbolAddress, taken once per device in
// nda_create with that device current, and is kept in g_scratch.
static __device__ __align__(256) uint8_t scratch[NDA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch[MAX_DEVICES] = {};

// This device's address of `scratch` (resolved on first use per device).
hipError_t scratch_address(int dev, uint8_t **out)
{
    if (dev < 0 || dev >= MAX_DEVICES)
        return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return e;
        g_scratch[dev] = static_cast<uint8_t *>(p);
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

// Device memory of every context, CQ tensor and nda_dev_alloc block comes
// from this pair (the engine's ND_ALLOC / ND_FREE seam, nd_model.h:35-68);
// nda_set_allocator replaces it.
void *default_alloc(size_t bytes, void *)
{
    void *p = nullptr;
    return hipMalloc(&p, bytes) == hipSuccess ? p : nullptr;
}
void default_free(void *p, void *) { (void)hipFree(p); }

std::mutex g_alloc_mu;
nda_alloc_fn g_alloc = default_alloc;
nda_free_fn g_free = default_free;
void *g_alloc_user = nullptr;

void *dev_alloc(size_t bytes)
{
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    return g_alloc(bytes ? bytes : 1, g_alloc_user);
}

void dev_free(void *p)
{
    if (!p)
        return;
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    g_free(p, g_alloc_user);
}

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

} // namespace

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

namespace {

int fail(nda_ctx *c, int code, const char *fmt, ...)
{
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return code;
}

int hip_fail(nda_ctx *c, hipError_t e, const char *what)
{
    return fail(c, e == hipErrorOutOfMemory ? NDA_ERR_NOMEM : NDA_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
}

#define HIPC(c, call)                                      \
    do {                                                   \
        hipError_t e_ = (call);                            \
        if (e_ != hipSuccess)                              \
            return hip_fail((c), e_, #call);               \
    } while (0)

// Calls on one context are ordered as if they ran on one stream. A call
// rewrites device tables and scratch buffers (sequence and page tables, row
// staging, work lists, split partials, block scratch) that the previous
// call's kernels may still be reading; so a call on a stream other than the
// previous call's first makes its stream wait for everything queued on the
// previous one (an event recorded there), before it uploads or launches
// anything. Calls on one stream need nothing: stream order covers them.
int on_stream(nda_ctx *c, hipStream_t st)
{
    if (c->has_stream && c->last_stream != st) {
        HIPC(c, hipEventRecord(c->order_ev, c->last_stream));
        HIPC(c, hipStreamWaitEvent(st, c->order_ev, 0));
    }
    c->last_stream = st;
    c->has_stream = true;
    return NDA_OK;
}

// Host-to-device upload of n bytes on stream st, returning without waiting
// for the stream. A copy from pageable memory blocks the caller until the
// stream reaches it, which would keep the host from running ahead of the GPU
// at every call; so the bytes are copied into the context's pinned ring and
// sent from there. A region of the ring is written again only after the
// event recorded behind its last copy has completed (the oldest uploads are
// waited for when the ring wraps onto them), and the events are the
// context's own (created with it): an upload allocates nothing. The caller's
// buffer may be reused as soon as this returns.
int upload(nda_ctx *c, void *dst, const void *src, size_t n, hipStream_t st)
{
    if (n == 0)
        return NDA_OK;
    const size_t need = (n + 255) & ~(size_t)255;
    if (!c->h_ring || need > c->ring_cap / 2) {
        HIPC(c, hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, st));
        return NDA_OK;
    }
    if (c->ring_head + need > c->ring_cap)
        c->ring_head = 0;
    const size_t lo = c->ring_head, hi = lo + need;
    auto retire_front = [&](bool wait) -> hipError_t {
        UploadRec &u = c->ring_live[c->live_head];
        const hipError_t e = wait ? hipEventSynchronize(u.ev) : hipEventQuery(u.ev);
        if (e == hipSuccess) {
            c->ring_ev.push_back(u.ev);          // within the reserved capacity
            c->live_head = (c->live_head + 1) % UPLOAD_EVENTS;
            c->live_n--;
        }
        return e;
    };
    // completed uploads give their regions and events back
    while (c->live_n && retire_front(false) == hipSuccess) {
    }
    // the oldest uploads are waited for while one still overlaps [lo, hi),
    // or while no event is free
    for (;;) {
        bool blocked = c->ring_ev.empty();
        for (int i = 0; i < c->live_n && !blocked; i++) {
            const UploadRec &u = c->ring_live[(c->live_head + i) % UPLOAD_EVENTS];
            blocked = u.lo < hi && lo < u.hi;
        }
        if (!blocked)
            break;
        if (hipError_t e = retire_front(true); e != hipSuccess)
            return hip_fail(c, e, "hipEventSynchronize (upload ring)");
    }
    memcpy(c->h_ring + lo, src, n);
    HIPC(c, hipMemcpyAsync(dst, c->h_ring + lo, n, hipMemcpyHostToDevice, st));
    hipEvent_t ev = c->ring_ev.back();
    HIPC(c, hipEventRecord(ev, st));
    c->ring_ev.pop_back();
    c->ring_live[(c->live_head + c->live_n) % UPLOAD_EVENTS] = UploadRec{lo, hi, ev};
    c->live_n++;
    c->ring_head = hi;
    return NDA_OK;
}

void release_pages(nda_ctx *c, uint32_t seq) { c->pt.release(seq); }

// Back own slots [s0, s1) of a sequence with pages. All-or-nothing.
int back_slots(nda_ctx *c, uint32_t seq, uint32_t s0, uint32_t s1)
{
    if (!c->pt.back_slots(seq, s0, s1))
        return fail(c, NDA_ERR_NOMEM, "page pool exhausted: need %zu pages, %zu free", c->pt.need(seq, s0, s1),
                    c->pt.free_pages.size());
    return NDA_OK;
}

// Back the own slot(s) of positions [p0, p0 + n) (no wrap inside, n >= 1);
// pages an earlier run took before the pool ran out stay until the caller's
// transaction gives them back.
int back_positions(nda_ctx *c, uint32_t seq, uint32_t p0, uint32_t n)
{
    if (!c->pt.back_positions(seq, c->seqs[seq], p0, n, c->pg.window))
        return fail(c, NDA_ERR_NOMEM, "page pool exhausted (sequence %u, %zu pages free)", seq,
                    c->pt.free_pages.size());
    return NDA_OK;
}

int sync_tables(nda_ctx *c, hipStream_t st)
{
    if (c->seqs_dirty) {
        std::vector<SeqDev> tmp(c->seqs.size());
        for (size_t i = 0; i < tmp.size(); i++) {
            tmp[i].pos = (int32_t)c->seqs[i].pos;
            tmp[i].n_sink = (int32_t)c->seqs[i].n_sink;
            tmp[i].prefix = c->seqs[i].prefix;
            tmp[i].pad = 0;
        }
        if (int rc = upload(c, c->d_seqs, tmp.data(), tmp.size() * sizeof(SeqDev), st))
            return rc;
        c->seqs_dirty = false;
    }
    if (c->pt.dirty_lo < c->pt.dirty_hi) {
        size_t off = (size_t)c->pt.dirty_lo * c->pg.pages_per_seq;
        size_t n = (size_t)(c->pt.dirty_hi - c->pt.dirty_lo) * c->pg.pages_per_seq;
        if (int rc = upload(c, c->d_pages + off, c->pt.pages.data() + off, n * sizeof(int32_t), st))
            return rc;
        c->pt.dirty_lo = UINT32_MAX;
        c->pt.dirty_hi = 0;
    }
    if (c->pt.prefix_dirty) {
        if (int rc = upload(c, c->d_prefix_pages, c->pt.prefix_pages.data(),
                            c->pt.prefix_pages.size() * sizeof(int32_t), st))
            return rc;
        c->pt.prefix_dirty = false;
    }
    return NDA_OK;
}

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

// row_seq | row_t staging for `rows` rows
int ensure_rows(nda_ctx *c, size_t rows)
{
    return grow_buf(c, c->d_rows, c->rows_cap, rows * 2, std::max<size_t>(rows * 2, 8192));
}

int ensure_part(nda_ctx *c, size_t floats) { return grow_buf(c, c->d_part, c->part_cap, floats, floats); }

int ensure_pf(nda_ctx *c, size_t n) { return grow_buf(c, c->d_pf, c->pf_cap, n, std::max<size_t>(n * 2, 16384)); }

int ensure_stage(nda_ctx *c, size_t bytes) { return grow_buf(c, c->d_stage, c->stage_cap, bytes, bytes); }

template <typename T>
int ensure_buf(nda_ctx *c, T *&buf, size_t &cap, size_t need)
{
    return grow_buf(c, buf, cap, need, std::max<size_t>(need, 4096));
}

hipEvent_t take_event(nda_ctx *c)
{
    if (!c->ev_free.empty()) {
        hipEvent_t e = c->ev_free.back();
        c->ev_free.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

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

int check_seq(nda_ctx *c, uint32_t seq)
{
    if (seq >= c->cfg.max_seqs)
        return fail(c, NDA_ERR_ARG, "sequence %u out of range (max_seqs %u)", seq, c->cfg.max_seqs);
    return NDA_OK;
}

int check_ids(nda_ctx *c, uint32_t nseq, const uint32_t *ids)
{
    if (nseq > c->cfg.max_seqs)
        return fail(c, NDA_ERR_ARG, "nseq %u > max_seqs %u", nseq, c->cfg.max_seqs);
    if (ids)
        for (uint32_t b = 0; b < nseq; b++)
            if (ids[b] >= c->cfg.max_seqs)
                return fail(c, NDA_ERR_ARG, "seq_ids[%u] = %u out of range", b, ids[b]);
    return NDA_OK;
}

inline uint32_t sid(const uint32_t *ids, uint32_t b) { return ids ? ids[b] : b; }

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// ---- tap histories of the attention front ----

float *hist_live(nda_ctx *c, uint32_t seq) { return c->d_hist + (uint64_t)seq * c->hist_block; }
float *hist_snap(nda_ctx *c, uint32_t seq) { return c->d_snap_hist + (uint64_t)seq * c->hist_block; }
float *hist_prefix(nda_ctx *c, int32_t id) { return c->d_prefix_hist + (uint64_t)id * c->hist_block; }

// Queue a whole-block copy (src null: clear). Calls without a stream
// (reset, rewind) only queue; the queue is applied in order on the caller's
// stream before the next front launch or history read.
int hist_flush(nda_ctx *c, hipStream_t st);

void hist_queue(nda_ctx *c, float *dst, const float *src)
{
    if (!c->taps)
        return;
    c->hist_pending.push_back({dst, src});
    // A context that never runs the front again would only grow the queue:
    // past this length it is applied on the stream of the context's last
    // call (stream order then covers it).
    if (c->hist_pending.size() >= (1u << 16))
        (void)hist_flush(c, c->has_stream ? c->last_stream : nullptr);
}

int hist_flush(nda_ctx *c, hipStream_t st)
{
    if (c->hist_pending.empty())
        return NDA_OK;
    const size_t n = c->hist_pending.size();
    if (int rc = ensure_buf(c, c->d_hist_ops, c->hist_ops_cap, n))
        return rc;
    if (int rc = upload(c, c->d_hist_ops, c->hist_pending.data(), n * sizeof(HistOp), st))
        return rc;
    // Launch maximal runs of ops that touch disjoint blocks; a run ends where
    // an op writes a block the run reads or writes, or reads one it writes.
    std::unordered_set<const float *> dsts, srcs;
    size_t b0 = 0;
    auto launch = [&](size_t b1) -> int {
        for (size_t o = b0; o < b1; o += 65535) {
            hipError_t e = launch_hist_ops(c->d_hist_ops + o, (uint32_t)std::min<size_t>(65535, b1 - o),
                                           c->hist_block, st);
            if (e != hipSuccess)
                return hip_fail(c, e, "history copy launch");
        }
        return NDA_OK;
    };
    for (size_t i = 0; i < n; i++) {
        const HistOp &op = c->hist_pending[i];
        const bool clash = dsts.count(op.dst) || srcs.count(op.dst) || (op.src && dsts.count(op.src));
        if (clash) {
            if (int rc = launch(i))
                return rc;
            b0 = i;
            dsts.clear();
            srcs.clear();
        }
        dsts.insert(op.dst);
        if (op.src)
            srcs.insert(op.src);
    }
    if (int rc = launch(n))
        return rc;
    c->hist_pending.clear();
    return NDA_OK;
}

// Room on the device for `extra` more queued history copies, taken before a
// call changes any state (so a failed allocation changes nothing).
int hist_reserve(nda_ctx *c, size_t extra)
{
    if (!c->taps)
        return NDA_OK;
    return ensure_buf(c, c->d_hist_ops, c->hist_ops_cap, c->hist_pending.size() + extra);
}

// Upload seq ids (and optional per-row offsets) for a launch; returns device
// pointers, null when the identity mapping applies.
int upload_rows(nda_ctx *c, uint32_t rows, const uint32_t *row_seq, const uint32_t *row_t,
                hipStream_t st, const uint32_t **d_seq, const uint32_t **d_t)
{
    *d_seq = nullptr;
    *d_t = nullptr;
    if (!row_seq && !row_t)
        return NDA_OK;
    int rc = ensure_rows(c, rows);
    if (rc)
        return rc;
    if (row_seq) {
        if (int rc2 = upload(c, c->d_rows, row_seq, rows * sizeof(uint32_t), st))
            return rc2;
        *d_seq = c->d_rows;
    }
    if (row_t) {
        if (int rc2 = upload(c, c->d_rows + rows, row_t, rows * sizeof(uint32_t), st))
            return rc2;
        *d_t = c->d_rows + rows;
    }
    return NDA_OK;
}

// Split-KV size for a launch. With enough (row, kv-head) units to fill the
// chip many times over, rows are not split (no partials, no merge); with few
// units, rows are cut into chunks so that ~64 work items per CU balance the
// ragged lengths, but never below 1024 positions, where the merge launch
// would cost more than the split saves (one engine session at a few hundred
// positions runs as one launch). A fixed split_chunk in the config overrides
// this.
uint32_t pick_chunk(const nda_ctx *c, uint64_t units, uint64_t sum_total, uint32_t max_total)
{
    if (c->chunk)
        return c->chunk;
    const uint64_t cus = (uint64_t)c->cus;
    uint64_t ch;
    if (units >= 16 * cus)
        ch = std::max<uint64_t>(max_total, 64);
    else
        ch = std::max<uint64_t>(1024, (sum_total * c->cfg.n_kv_heads / (64 * cus) + 63) / 64 * 64);
    // grid.y bound
    const uint64_t min_ch = ((uint64_t)max_total + 65534) / 65535;
    ch = std::max(ch, min_ch);
    return (uint32_t)std::min<uint64_t>(ch, 1u << 30);
}

AttnArgs attn_args(nda_ctx *c, uint32_t layer, uint32_t rows, const float *q, const float *gate,
                   float *out, uint32_t max_total, uint64_t sum_total)
{
    AttnArgs a{};
    a.q = q;
    a.gate = gate;
    a.out = out;
    a.pool = c->pool + (uint64_t)layer * c->pg.layer_bytes;
    a.page_table = c->d_pages;
    a.prefix_pages = c->d_prefix_pages;
    a.seqs = c->d_seqs;
    a.part = c->d_part;
    a.pg = c->pg;
    a.rows = rows;
    a.nh = c->cfg.n_heads;
    a.chunk = pick_chunk(c, (uint64_t)rows * c->cfg.n_kv_heads, sum_total, max_total);
    // grid.y and the partial-buffer stride: chunks of the longest row.
    a.max_chunks = std::max<uint32_t>(1, (max_total + a.chunk - 1) / a.chunk);
    a.qscale = (float)(1.4426950408889634 / std::sqrt((double)c->cfg.qk_head_dim));
    a.avg_len = rows ? (uint32_t)std::min<uint64_t>(sum_total / rows, 0xFFFFFFFFu) : 0;
    return a;
}

// GQA decode on MFMA: with 4 or more query heads per kv-head (int8 K/V),
// one wave per (row, kv-head) runs the prefill kernel's tile arithmetic with
// the group's heads as its rows (S^T = K.Q^T, O^T += V^T.P^T), where the
// VALU kernel spends its time on per-lane dot products and their lane
// reductions (2.5x on 4096 rows of the engine's 12/2-head shape). Launches
// that fuse the store, carry per-row offsets or split rows stay on the VALU
// kernel, and so do tiny ones (an engine session), whose VALU waves split
// each row's positions between them.
constexpr uint64_t MFMA_DECODE_MIN_ITEMS = 16;

bool mfma_decode_geo(const nda_ctx *c)
{
    return decode_mfma_supported(c->geo) && !(c->cfg.flags & NDA_FLAG_DECODE_VALU);
}

bool mfma_decode(const nda_ctx *c, const AttnArgs &a)
{
    return mfma_decode_geo(c) && !a.k_new && !a.row_t && a.max_chunks == 1 &&
           (uint64_t)a.rows * c->cfg.n_kv_heads >= MFMA_DECODE_MIN_ITEMS;
}

// Device buffers an attention launch over `rows` rows needs: the row staging
// (staged: ids or per-row offsets are uploaded) and, for rows split into
// chunks (which the VALU kernel serves), the partials. Taken before a call
// changes any state, so that a failed allocation changes nothing.
int reserve_attend(nda_ctx *c, uint32_t rows, bool staged, uint32_t max_total, uint64_t sum_total)
{
    if (staged)
        if (int rc = ensure_rows(c, rows))
            return rc;
    const AttnArgs a = attn_args(c, 0, rows, nullptr, nullptr, nullptr, max_total, sum_total);
    if (a.max_chunks > 1)
        return ensure_part(c, (size_t)a.rows * a.nh * a.max_chunks * (c->cfg.v_head_dim + 2));
    return NDA_OK;
}

// The GQA decode's work order for the batch of sequences 0..rows-1: rows by
// key tiles visited, most first (a counting sort). Its waves then finish
// together: in row order the ragged tail of the last waves cost 3% of the
// launch. Built once per change of sequence state (the 8 layers of a step
// share it) and uploaded on the caller's stream; any permutation of the rows
// gives the same results, so a stale order only costs time. A failed
// allocation just leaves the rows in order.
static const uint32_t *decode_order(nda_ctx *c, uint32_t rows, hipStream_t st)
{
    if (c->d_order && c->order_rows == rows && c->order_ver == c->state_ver)
        return c->d_order;
    std::vector<uint32_t> tiles(rows), first;
    uint32_t top = 0;
    for (uint32_t b = 0; b < rows; b++) {
        const SeqHost &s = c->seqs[b];
        const Vis v = visible(s, s.pos, c->cfg.window);
        tiles[b] = (v.n_sh + 31) / 32 + (v.n_own + 31) / 32;
        top = std::max(top, tiles[b]);
    }
    first.assign(top + 2, 0u);
    for (uint32_t b = 0; b < rows; b++)         // counts, then starts, by descending tiles
        first[top - tiles[b] + 1]++;
    for (uint32_t k = 1; k <= top + 1; k++)
        first[k] += first[k - 1];
    std::vector<uint32_t> ord(rows);
    for (uint32_t b = 0; b < rows; b++)
        ord[first[top - tiles[b]]++] = b;
    if (grow_buf(c, c->d_order, c->order_cap, rows, std::max<size_t>(rows, 4096)) ||
        upload(c, c->d_order, ord.data(), (size_t)rows * 4, st)) {
        c->order_rows = 0;
        return nullptr;
    }
    c->order_rows = rows;
    c->order_ver = c->state_ver;
    return c->d_order;
}

// part: split-KV partials of at least rows * nh * max_chunks * (v_hd + 2)
// floats, or null for the context's own buffer (grown on demand). prof: record
// profiling events (nda_decode_noalloc records none: creating an event may
// allocate). ordered: the GQA decode may take the rows longest first (it then
// builds or reuses the context's order buffer; nda_decode_noalloc does not).
int run_attend(nda_ctx *c, AttnArgs &a, hipStream_t st, float *part = nullptr, bool prof = true,
               bool ordered = true)
{
    if (mfma_decode(c, a)) {
        PrefillArgs pa{};
        pa.q = a.q;
        pa.gate = a.gate;
        pa.out = a.out;
        pa.pool = a.pool;
        pa.page_table = a.page_table;
        pa.prefix_pages = a.prefix_pages;
        pa.seqs = a.seqs;
        pa.row_seq = a.row_seq;
        pa.pg = a.pg;
        pa.n_items = a.rows * c->cfg.n_kv_heads;
        pa.nh = a.nh;
        pa.qscale = a.qscale;
        // enough rows for several rounds of waves, rows 0..rows-1
        if (ordered && !a.row_seq && pa.n_items >= 4u * (uint32_t)c->cus)
            pa.items = decode_order(c, a.rows, st);
        ProfScope ps(c, NDA_K_DECODE, st, prof);
        hipError_t e = launch_decode_mfma(c->geo, pa, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "decode (MFMA) kernel launch");
        return NDA_OK;
    }
    if (a.max_chunks > 1) {
        if (part) {
            a.part = part;
        } else {
            int rc = ensure_part(c, (size_t)a.rows * a.nh * a.max_chunks * (c->cfg.v_head_dim + 2));
            if (rc)
                return rc;
            a.part = c->d_part;
        }
    }
    {
        ProfScope ps(c, NDA_K_DECODE, st, prof);
        hipError_t e = launch_attend(c->geo, a, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "attend kernel launch");
    }
    if (a.max_chunks > 1 && !(a.chunk_lo == 1 && a.max_chunks == 2)) {
        ProfScope ps(c, NDA_K_COMBINE, st, prof);
        hipError_t e = launch_combine(c->geo, a, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "combine kernel launch");
    }
    return NDA_OK;
}

} // namespace

// ===================================================================== ABI

extern "C" {

int nda_create(const nda_config *cfg_in, nda_ctx **out)
{
    if (!cfg_in || !out)
        return NDA_ERR_ARG;
    *out = nullptr;
    nda_config cfg = *cfg_in;
    if (cfg.page_size == 0)
        cfg.page_size = 16;
    if (cfg.max_prefixes == 0)
        cfg.max_prefixes = 16;
    if (!cfg.n_layers || !cfg.n_heads || !cfg.n_kv_heads || cfg.n_heads % cfg.n_kv_heads ||
        !cfg.window || !cfg.max_seqs || cfg.kv_dtype > NDA_KV_F16)
        return NDA_ERR_ARG;
    if (cfg.page_size != 16 && cfg.page_size != 32 && cfg.page_size != 64)
        return NDA_ERR_ARG;
    if (cfg.window > (1u << 30))
        return NDA_ERR_ARG;
    Geo geo{(int)(cfg.kv_dtype == NDA_KV_F16), (int)cfg.qk_head_dim, (int)cfg.v_head_dim,
            (int)(cfg.n_heads / cfg.n_kv_heads)};
    if (!geometry_supported(geo))
        return NDA_ERR_UNSUPPORTED;

    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return NDA_ERR_NODEV;

    nda_ctx *c = new (std::nothrow) nda_ctx();
    if (!c)
        return NDA_ERR_NOMEM;
    c->cfg = cfg;
    c->geo = geo;
    const uint32_t P = cfg.page_size;
    uint32_t lg = 0;
    while ((1u << lg) < P)
        lg++;
    const uint64_t es = cfg.kv_dtype == NDA_KV_F16 ? 2 : 1;
    c->pg.log2_page = lg;
    c->pg.pages_per_seq = (cfg.window + P - 1) / P;
    c->pg.head_bytes = (uint64_t)P * (cfg.qk_head_dim + cfg.v_head_dim) * es + (es == 1 ? 8ull * P : 0ull);
    c->pg.page_bytes = c->pg.head_bytes * cfg.n_kv_heads;
    c->pg.window = cfg.window;
    c->pg.nkv = cfg.n_kv_heads;
    c->pg.dk = cfg.qk_head_dim;
    c->pg.dv = cfg.v_head_dim;
    c->max_pages = cfg.max_pages ? cfg.max_pages
                                 : (uint64_t)(cfg.max_seqs + cfg.max_prefixes) * c->pg.pages_per_seq;
    if (c->max_pages > (uint64_t)INT32_MAX) {
        delete c;
        return NDA_ERR_ARG;
    }
    c->pg.layer_bytes = c->pg.page_bytes * c->max_pages;

    // Split-KV: a sequence longer than `chunk` visible positions is split into
    // chunks merged by the combine kernel. Visible positions <= 2 * window
    // (shared sinks + own slots).
    c->chunk = cfg.split_chunk;
    if (c->chunk % 64)
        c->chunk = (c->chunk + 63) / 64 * 64;
    if (c->chunk && (2ull * cfg.window + c->chunk - 1) / c->chunk > 65535) {
        delete c;
        return NDA_ERR_ARG;
    }
    {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess &&
            prop.multiProcessorCount > 0)
            c->cus = prop.multiProcessorCount;
        // the device's nda_decode_noalloc scratch, with this device current
        if (hipGetDevice(&dev) != hipSuccess || scratch_address(dev, &c->scratch) != hipSuccess) {
            delete c;
            return NDA_ERR_HIP;
        }
    }

    const uint64_t pool_bytes = c->pg.layer_bytes * cfg.n_layers;
    c->pool = static_cast<uint8_t *>(dev_alloc(pool_bytes));
    if (!c->pool) {
        delete c;
        return NDA_ERR_NOMEM;
    }
    c->dev_bytes = pool_bytes;
    const size_t pt = (size_t)cfg.max_seqs * c->pg.pages_per_seq;
    const size_t ppt = (size_t)cfg.max_prefixes * c->pg.pages_per_seq;
    c->d_pages = static_cast<int32_t *>(dev_alloc(pt * 4));
    c->d_prefix_pages = static_cast<int32_t *>(dev_alloc(ppt * 4));
    c->d_seqs = static_cast<SeqDev *>(dev_alloc((size_t)cfg.max_seqs * sizeof(SeqDev)));
    if (!c->d_pages || !c->d_prefix_pages || !c->d_seqs) {
        nda_destroy(c);
        return NDA_ERR_NOMEM;
    }
    c->dev_bytes += pt * 4 + ppt * 4 + (size_t)cfg.max_seqs * sizeof(SeqDev);
    if (hipEventCreateWithFlags(&c->order_ev, hipEventDisableTiming) != hipSuccess) {
        c->order_ev = nullptr;
        nda_destroy(c);
        return NDA_ERR_HIP;
    }
    // the pinned upload ring and its events; without them uploads copy from
    // pageable memory (correct, but the host then waits for the stream)
    if (hipHostMalloc((void **)&c->h_ring, UPLOAD_RING_BYTES, hipHostMallocDefault) == hipSuccess) {
        // every page touched once here: the first pass of uploads through
        // untouched ring pages ran ~15x slower (0.44 against 0.03 ms for
        // one layer's tables), which put milliseconds into the first calls
        memset(c->h_ring, 0, UPLOAD_RING_BYTES);
        c->ring_cap = UPLOAD_RING_BYTES;
        c->ring_ev.reserve(UPLOAD_EVENTS);
        for (int i = 0; i < UPLOAD_EVENTS; i++) {
            hipEvent_t e;
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
                break;
            c->ring_ev.push_back(e);
        }
        if (c->ring_ev.empty()) {
            (void)hipHostFree(c->h_ring);
            c->h_ring = nullptr;
            c->ring_cap = 0;
        }
    } else {
        c->h_ring = nullptr;
        (void)hipGetLastError();
    }
    try {
        c->pt.init(cfg.max_seqs, cfg.max_prefixes, c->pg.pages_per_seq, c->pg.log2_page, c->max_pages);
        c->seqs.assign(cfg.max_seqs, SeqHost());
        c->prefixes.assign(cfg.max_prefixes, Prefix());
    } catch (...) {
        nda_destroy(c);
        return NDA_ERR_NOMEM;
    }
    *out = c;
    return NDA_OK;
}

void nda_destroy(nda_ctx *c)
{
    if (!c)
        return;
    (void)hipDeviceSynchronize();
    for (auto &r : c->prof_pending) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->ev_free)
        (void)hipEventDestroy(e);
    for (int i = 0; i < c->live_n; i++)
        (void)hipEventDestroy(c->ring_live[(c->live_head + i) % UPLOAD_EVENTS].ev);
    for (auto e : c->ring_ev)
        (void)hipEventDestroy(e);
    if (c->order_ev)
        (void)hipEventDestroy(c->order_ev);
    if (c->h_ring)
        (void)hipHostFree(c->h_ring);
    void *bufs[] = {c->pool, c->d_pages, c->d_prefix_pages, c->d_seqs, c->d_rows, c->d_part,
                    c->d_stage, c->d_pf, c->d_hist, c->d_snap_hist, c->d_prefix_hist,
                    c->d_front_w, c->d_front_norm, c->d_rope, c->d_qfront, c->d_front_rows,
                    c->d_hist_ops, c->d_bscr, c->d_order};
    for (void *b : bufs)
        dev_free(b);
    delete c;
}

const char *nda_last_error(const nda_ctx *c) { return c ? c->err.c_str() : "null context"; }

uint64_t nda_device_bytes(const nda_ctx *c) { return c ? c->dev_bytes : 0; }

int nda_seq_reset(nda_ctx *c, uint32_t seq)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    SeqHost &s = c->seqs[seq];
    if (s.prefix >= 0)
        c->prefixes[s.prefix].refs--;
    release_pages(c, seq);
    s = SeqHost();
    c->state_ver++;
    c->seqs_dirty = true;
    if (c->taps)
        hist_queue(c, hist_live(c, seq), nullptr);    // nd_model_reset, nd_model.c:1575-1580
    return NDA_OK;
}

int nda_seq_set_sink(nda_ctx *c, uint32_t seq, uint32_t n)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    SeqHost &s = c->seqs[seq];
    if (s.prefix >= 0)
        return fail(c, NDA_ERR_STATE, "sequence %u reads its sinks from prefix %d", seq, s.prefix);
    s.n_sink = clamp_sink(c->cfg.window, n);
    c->state_ver++;
    c->seqs_dirty = true;
    return NDA_OK;
}

int nda_seq_state(const nda_ctx *c, uint32_t seq, uint32_t *pos, uint32_t *n_sink, int32_t *prefix_id)
{
    if (!c || seq >= c->cfg.max_seqs)
        return NDA_ERR_ARG;
    const SeqHost &s = c->seqs[seq];
    if (pos)
        *pos = s.pos;
    if (n_sink)
        *n_sink = s.n_sink;
    if (prefix_id)
        *prefix_id = s.prefix;
    return NDA_OK;
}

int nda_seq_set_pos(nda_ctx *c, uint32_t seq, uint32_t pos)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    SeqHost &s = c->seqs[seq];
    if (s.prefix >= 0 && pos < s.n_sink)
        return fail(c, NDA_ERR_RANGE, "pos %u inside the shared prefix (%u)", pos, s.n_sink);
    s.pos = pos;
    c->state_ver++;
    c->seqs_dirty = true;
    return NDA_OK;
}

int nda_seq_reserve(nda_ctx *c, uint32_t seq, uint32_t n)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    if (n == 0)
        return NDA_OK;
    const SeqHost &s = c->seqs[seq];
    // Once the ring is full every slot is backed; cap at one full cycle.
    uint32_t cap = c->cfg.window - (s.prefix >= 0 ? s.n_sink : 0);
    PageTxn txn(c->pt);
    if (int rc = back_positions(c, seq, s.pos, std::min(n, cap)))
        return rc;
    txn.commit();
    return NDA_OK;
}

int nda_advance(nda_ctx *c, uint32_t nseq, const uint32_t *ids, uint32_t n, void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    if (nseq == 0 || n == 0)
        return NDA_OK;
    if (!c->seqs_dirty && ids)
        if (int rc = ensure_rows(c, nseq))
            return rc;
    for (uint32_t b = 0; b < nseq; b++)
        c->seqs[sid(ids, b)].pos += n;
    c->state_ver++;
    if (c->seqs_dirty)      // a full upload is pending anyway
        return NDA_OK;
    // Same increment on the device copy, in stream order, so steady-state
    // decoding uploads nothing.
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    const uint32_t *d_seq, *d_t;
    if (int rc = upload_rows(c, nseq, ids, nullptr, st, &d_seq, &d_t))
        return rc;
    hipError_t e = launch_advance(c->d_seqs, d_seq, nseq, n, st);
    if (e != hipSuccess)
        return hip_fail(c, e, "advance kernel launch");
    return NDA_OK;
}

int nda_prefix_build(nda_ctx *c, uint32_t seq, int32_t *prefix_id, void *stream)
{
    if (!c || !prefix_id)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    SeqHost &s = c->seqs[seq];
    const uint32_t len = s.pos;
    if (len == 0)
        return fail(c, NDA_ERR_STATE, "sequence %u holds no positions", seq);
    if (len > c->cfg.window)
        return fail(c, NDA_ERR_RANGE, "prefix of %u positions exceeds the window %u", len, c->cfg.window);
    int32_t id = -1;
    for (uint32_t i = 0; i < c->cfg.max_prefixes; i++)
        if (!c->prefixes[i].used) {
            id = (int32_t)i;
            break;
        }
    if (id < 0)
        return fail(c, NDA_ERR_NOMEM, "all %u prefix segments in use", c->cfg.max_prefixes);
    const uint32_t npages = (len + c->cfg.page_size - 1) / c->cfg.page_size;
    if (npages > c->pt.free_pages.size())
        return fail(c, NDA_ERR_NOMEM, "page pool exhausted building a prefix");
    if (int rc = hist_reserve(c, 2))
        return rc;
    c->pt.take_prefix(id, npages);
    if (int rc = sync_tables(c, st))
        return rc;

    // Copy positions [0, len): shared part (if this sequence is itself
    // attached) then its own slots (no wrap: len <= window).
    const Vis v = visible(s, len - 1, c->cfg.window);
    CopyArgs ca{};
    ca.pool = c->pool;
    ca.n_layers = c->cfg.n_layers;
    ca.pg = c->pg;
    ca.dst_pages = c->d_prefix_pages + (size_t)id * c->pg.pages_per_seq;
    if (v.n_sh) {
        ca.src_pages = c->d_prefix_pages + (size_t)s.prefix * c->pg.pages_per_seq;
        ca.src_slot0 = 0;
        ca.dst_slot0 = 0;
        ca.count = v.n_sh;
        hipError_t e = launch_copy(c->geo, ca, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "prefix copy");
    }
    if (v.n_own) {
        ca.src_pages = c->d_pages + (size_t)seq * c->pg.pages_per_seq;
        ca.src_slot0 = 0;
        ca.dst_slot0 = v.n_sh;
        ca.count = v.n_own;
        hipError_t e = launch_copy(c->geo, ca, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "prefix copy");
    }
    Prefix &pf = c->prefixes[id];
    pf.used = true;
    pf.len = len;
    pf.n_sink = clamp_sink(c->cfg.window, len);
    pf.refs = 0;
    // nd_model_snapshot: the builder pins its own positions as sinks.
    if (s.prefix < 0)
        s.n_sink = pf.n_sink;
    c->state_ver++;
    s.has_snap = true;
    s.snap_pos = len;
    c->seqs_dirty = true;
    *prefix_id = id;
    // The tap histories go with the snapshot and the prefix
    // (nd_model.c:1423-1425, :1519-1521).
    if (c->taps) {
        hist_queue(c, hist_prefix(c, id), hist_live(c, seq));
        hist_queue(c, hist_snap(c, seq), hist_live(c, seq));
        if (int rc = hist_flush(c, st))
            return rc;
    }
    return NDA_OK;
}

int nda_seq_attach(nda_ctx *c, uint32_t seq, int32_t id, void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    if (id < 0 || (uint32_t)id >= c->cfg.max_prefixes || !c->prefixes[id].used)
        return fail(c, NDA_ERR_ARG, "prefix %d does not exist", id);
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    SeqHost &s = c->seqs[seq];
    const Prefix &pf = c->prefixes[id];
    {
        // the ring tail's pages, from the free pool plus this sequence's own
        const uint32_t tail = pf.len > pf.n_sink ? pf.len - pf.n_sink : 0u;
        const size_t need = (tail + c->cfg.page_size - 1) / c->cfg.page_size;
        const size_t have = c->pt.free_pages.size() + c->pt.backed(seq);
        if (need > have)
            return fail(c, NDA_ERR_NOMEM, "page pool exhausted: need %zu pages, %zu free", need, have);
        if (int rc = hist_reserve(c, 2))
            return rc;
    }
    if (s.prefix >= 0)
        c->prefixes[s.prefix].refs--;
    release_pages(c, seq);
    s = SeqHost();
    c->state_ver++;
    s.prefix = id;
    s.n_sink = pf.n_sink;
    s.pos = pf.len;
    s.has_snap = true;
    s.snap_pos = pf.len;
    s.stored_end = pf.len;
    c->prefixes[id].refs++;
    c->seqs_dirty = true;
    if (c->taps) {   // nd_model_prefix_restore + rewind (nd_model.c:1543-1553, :1451-1453)
        hist_queue(c, hist_live(c, seq), hist_prefix(c, id));
        hist_queue(c, hist_snap(c, seq), hist_prefix(c, id));
        if (int rc = hist_flush(c, st))
            return rc;
    }
    // Positions past the sink clamp live in the ring: copy them in, as the
    // engine's restore copies every live slot.
    if (pf.len > pf.n_sink) {
        const uint32_t tail = pf.len - pf.n_sink;
        if (int rc = back_slots(c, seq, 0, tail))
            return rc;
        if (int rc = sync_tables(c, st))
            return rc;
        CopyArgs ca{};
        ca.pool = c->pool;
        ca.n_layers = c->cfg.n_layers;
        ca.pg = c->pg;
        ca.src_pages = c->d_prefix_pages + (size_t)id * c->pg.pages_per_seq;
        ca.dst_pages = c->d_pages + (size_t)seq * c->pg.pages_per_seq;
        ca.src_slot0 = pf.n_sink;
        ca.dst_slot0 = 0;
        ca.count = tail;
        hipError_t e = launch_copy(c->geo, ca, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "prefix tail copy");
    }
    return NDA_OK;
}

int nda_seq_rewind(nda_ctx *c, uint32_t seq)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    SeqHost &s = c->seqs[seq];
    if (!s.has_snap)
        return nda_seq_reset(c, seq);
    // Positions from snap_pos on are stored again from here; ring slots the
    // ring already overwrote stay lost (the inspection calls check both).
    const uint32_t rcap = c->cfg.window - s.n_sink;
    if (s.stored_end > rcap)
        s.ring_lo = std::max(s.ring_lo, s.stored_end - rcap);
    s.ring_lo = std::min(s.ring_lo, s.snap_pos);
    s.stored_end = std::min(s.stored_end, s.snap_pos);
    s.pos = s.snap_pos;
    c->state_ver++;
    c->seqs_dirty = true;
    if (c->taps)
        hist_queue(c, hist_live(c, seq), hist_snap(c, seq));   // nd_model.c:1451-1453
    return NDA_OK;
}

int nda_prefix_free(nda_ctx *c, int32_t id)
{
    if (!c)
        return NDA_ERR_ARG;
    if (id < 0 || (uint32_t)id >= c->cfg.max_prefixes || !c->prefixes[id].used)
        return fail(c, NDA_ERR_ARG, "prefix %d does not exist", id);
    if (c->prefixes[id].refs)
        return fail(c, NDA_ERR_STATE, "prefix %d is attached to %u sequences", id, c->prefixes[id].refs);
    c->pt.release_prefix(id);
    c->prefixes[id] = Prefix();
    return NDA_OK;
}

int nda_kv_append(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *k,
                  const float *v, void *stream)
{
    if (!c || (nseq && (!k || !v)))
        return c ? fail(c, NDA_ERR_ARG, "null k/v") : NDA_ERR_ARG;
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    if (ids)
        if (int rc = ensure_rows(c, nseq))
            return rc;
    PageTxn txn(c->pt);
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t q = sid(ids, b);
        if (int rc = back_positions(c, q, c->seqs[q].pos, 1))
            return rc;
    }
    txn.commit();
    for (uint32_t b = 0; b < nseq; b++) {
        SeqHost &s = c->seqs[sid(ids, b)];
        s.stored_end = std::max(s.stored_end, s.pos + 1);
    }
    if (int rc = sync_tables(c, st))
        return rc;
    const uint32_t *d_seq, *d_t;
    if (int rc = upload_rows(c, nseq, ids, nullptr, st, &d_seq, &d_t))
        return rc;
    AppendArgs a{};
    a.k = k;
    a.v = v;
    a.pool = c->pool + (uint64_t)layer * c->pg.layer_bytes;
    a.page_table = c->d_pages;
    a.seqs = c->d_seqs;
    a.row_seq = d_seq;
    a.row_t = d_t;
    a.pg = c->pg;
    a.rows = nseq;
    ProfScope ps(c, NDA_K_APPEND, st);
    hipError_t e = launch_append(c->geo, a, st);
    if (e != hipSuccess)
        return hip_fail(c, e, "append kernel launch");
    return NDA_OK;
}

// Decode, optionally with the append of this position fused in (k/v set).
// What nda_decode and nda_decode_noalloc check before any launch: arguments,
// and every visible slot backed (written by an append, a write or an attach;
// an unbacked one means the caller skipped the append). Returns the longest
// visible run and the sum over the listed sequences.
static int decode_check(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
                        float *out, uint32_t *max_total, uint64_t *sum_total)
{
    if (!c || (nseq && (!q || !out)))
        return c ? fail(c, NDA_ERR_ARG, "null q/out") : NDA_ERR_ARG;
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    *max_total = 0;
    *sum_total = 0;
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t qq = sid(ids, b);
        const SeqHost &s = c->seqs[qq];
        const Vis vv = visible(s, s.pos, c->cfg.window);
        *max_total = std::max(*max_total, vv.n_sh + vv.n_own);
        *sum_total += vv.n_sh + vv.n_own;
        if (vv.n_own) {
            const int32_t *row = &c->pt.pages[(size_t)qq * c->pg.pages_per_seq];
            if (row[(vv.n_own - 1) >> c->pg.log2_page] < 0 || row[0] < 0)
                return fail(c, NDA_ERR_STATE, "sequence %u: slot of position %u never stored", qq, s.pos);
        }
    }
    return NDA_OK;
}

// A decode batch whose sequences all read one shared prefix (the engine's
// requests on its routing schema) attends that prefix in one pass over all
// of them: per kv-head, the prefix's key tiles against every sequence's
// query rows on the prefill kernel's MFMA tiles, each row's softmax state
// left as its split-KV chunk 0 (chunks of n_sh positions). The VALU kernel
// continues with each sequence's own positions (chunks 1 on); a row of two
// chunks it merges with chunk 0 itself, longer rows go through the merge
// kernel. Without the pass the VALU kernel redoes the prefix's dot products
// for every sequence. Taken for batches of at least 4 (row,
// kv-head) units per CU of a shape the prefill kernel is built for and the
// MFMA GQA decode does not serve, with a prefix of at least one full key
// tile, and not when the append is fused into the launch. Rows longer than
// PREFIX_PASS_MAX_CHUNKS prefix lengths keep the single VALU pass: their own
// positions would be cut into many short work items (a prefix's length
// each), with partials and a merge, where the prefix is a small part of
// what they read.
struct PrefixSplit {
    bool on = false;
    int32_t prefix = -1;
    uint32_t n_sh = 0, max_chunks = 0, n_items = 0;
};
constexpr int PREFIX_PASS_WAVES = 2;    // 64-row work-groups: more of them to spread over the CUs
constexpr uint32_t PREFIX_PASS_MAX_CHUNKS = 4;

// whether a batch's sequences qualify (append not fused; see above)
static bool prefix_split_batch(const nda_ctx *c, uint32_t nseq, const uint32_t *ids, int32_t *pfx_out,
                               uint32_t *nsh_out)
{
    if (nseq == 0 || mfma_decode_geo(c) || !prefill_mfma_supported(c->geo) ||
        (c->cfg.flags & (NDA_FLAG_PREFILL_VALU | NDA_FLAG_DECODE_VALU)))
        return false;
    if ((uint64_t)nseq * c->cfg.n_kv_heads < 4ull * (uint64_t)c->cus)
        return false;
    int32_t pfx = -1;
    uint32_t nsh = 0;
    for (uint32_t b = 0; b < nseq; b++) {
        const SeqHost &s = c->seqs[sid(ids, b)];
        if (s.prefix < 0)
            return false;
        const Vis v = visible(s, s.pos, c->cfg.window);
        if (b == 0) {
            pfx = s.prefix;
            nsh = v.n_sh;
        } else if (s.prefix != pfx || v.n_sh != nsh) {
            return false;
        }
    }
    *pfx_out = pfx;
    *nsh_out = nsh;
    return nsh >= 32;
}

static void prefix_split_plan(nda_ctx *c, uint32_t nseq, const uint32_t *ids, bool fused, uint32_t max_total,
                              PrefixSplit &ps)
{
    ps = PrefixSplit();
    int32_t pfx;
    uint32_t nsh;
    if (fused || !prefix_split_batch(c, nseq, ids, &pfx, &nsh) || max_total <= nsh)
        return;
    const uint32_t chunks = (max_total + nsh - 1) / nsh;
    if (chunks > PREFIX_PASS_MAX_CHUNKS)
        return;
    ps.on = true;
    ps.prefix = pfx;
    ps.n_sh = nsh;
    ps.max_chunks = chunks;
    const uint64_t trows = 32u * PREFIX_PASS_WAVES;
    const uint64_t per_head = ((uint64_t)nseq * c->geo.rep + trows - 1) / trows;
    ps.n_items = (uint32_t)((per_head * c->cfg.n_kv_heads + 7) / 8 * 8);
}

// The prefix pass: work item (kv-head, tile of 64 rows of the batch), the
// rows being (sequence of the batch, query head of the group) pairs as the
// decode's q holds them.
static int prefix_pass(nda_ctx *c, const AttnArgs &a, uint32_t nseq, const uint32_t *ids, const PrefixSplit &ps,
                       hipStream_t st)
{
    const uint64_t trows = 32u * PREFIX_PASS_WAVES;
    const uint32_t per_head = (uint32_t)(((uint64_t)nseq * c->geo.rep + trows - 1) / trows);
    std::vector<uint32_t> items;
    items.reserve(8 * (size_t)ps.n_items);
    const uint32_t seq0 = sid(ids, 0);
    for (uint32_t g = 0; g < c->cfg.n_kv_heads; g++)
        for (uint32_t t = 0; t < per_head; t++) {
            // sequence, kv-head, row tile, first row, rows, position (unused),
            // prefix slots, prefix id; the sequence only names a page-table
            // row, which a pass with no own tiles never reads
            const uint32_t rec[8] = {seq0, g, t, 0u, nseq, ps.n_sh, ps.n_sh, (uint32_t)ps.prefix};
            items.insert(items.end(), rec, rec + 8);
        }
    while ((items.size() / 8) % 8) {
        const uint32_t pad[8] = {0xFFFFFFFFu, 0, 0, 0, 0, 0, 0, 0};
        items.insert(items.end(), pad, pad + 8);
    }
    if (int rc = upload(c, c->d_pf, items.data(), items.size() * 4, st))
        return rc;
    PrefillArgs pa{};
    pa.q = a.q;
    pa.pool = a.pool;
    pa.page_table = a.page_table;
    pa.prefix_pages = a.prefix_pages;
    pa.seqs = a.seqs;
    pa.items = c->d_pf;
    pa.part = a.part;
    pa.max_chunks = a.max_chunks;
    pa.tab_cap = (ps.n_sh + 31) / 32;         // the prefix's tiles only
    pa.pg = a.pg;
    pa.n_items = (uint32_t)(items.size() / 8);
    pa.nh = a.nh;
    pa.qscale = a.qscale;
    ProfScope ps_(c, NDA_K_DECODE, st);
    hipError_t e = launch_prefill(c->geo, pa, PREFIX_PASS_WAVES, st);
    if (e != hipSuccess)
        return hip_fail(c, e, "shared-prefix decode pass launch");
    return NDA_OK;
}

// The longest visible run and the sum over the listed sequences, at their
// current positions (valid ids).
static void decode_totals(const nda_ctx *c, uint32_t nseq, const uint32_t *ids, uint32_t *max_total,
                          uint64_t *sum_total)
{
    *max_total = 0;
    *sum_total = 0;
    for (uint32_t b = 0; b < nseq; b++) {
        const SeqHost &s = c->seqs[sid(ids, b)];
        const Vis vv = visible(s, s.pos, c->cfg.window);
        *max_total = std::max(*max_total, vv.n_sh + vv.n_own);
        *sum_total += vv.n_sh + vv.n_own;
    }
}

// The device buffers a decode of these sequences needs (row staging, split
// partials, the shared-prefix pass's partials and work list), grown before a
// call changes any state; psp: the shared-prefix pass plan.
static int decode_reserve(nda_ctx *c, uint32_t nseq, const uint32_t *ids, bool fused, uint32_t max_total,
                          uint64_t sum_total, PrefixSplit &psp)
{
    if (int rc = reserve_attend(c, nseq, ids != nullptr, max_total, sum_total))
        return rc;
    prefix_split_plan(c, nseq, ids, fused, max_total, psp);
    if (psp.on) {
        if (int rc = ensure_part(c, (size_t)nseq * c->cfg.n_heads * psp.max_chunks * (c->cfg.v_head_dim + 2)))
            return rc;
        if (int rc = ensure_pf(c, 8 * (size_t)psp.n_items))
            return rc;
    }
    return NDA_OK;
}

static int decode_impl(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
                       const float *k, const float *v, const float *gate, float *out, void *stream)
{
    if (c && nseq && k && !v)
        return fail(c, NDA_ERR_ARG, "null v");
    if (!c || (nseq && (!q || !out)))
        return c ? fail(c, NDA_ERR_ARG, "null q/out") : NDA_ERR_ARG;
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    // The fused store backs this position's slot first; the pages go back if
    // anything below fails.
    PageTxn txn(c->pt);
    if (k)
        for (uint32_t b = 0; b < nseq; b++) {
            const uint32_t qq = sid(ids, b);
            if (int rc = back_positions(c, qq, c->seqs[qq].pos, 1))
                return rc;
        }
    uint32_t max_total;
    uint64_t sum_total;
    if (int rc = decode_check(c, layer, nseq, ids, q, out, &max_total, &sum_total))
        return rc;
    PrefixSplit psp;
    if (int rc = decode_reserve(c, nseq, ids, k != nullptr, max_total, sum_total, psp))
        return rc;
    txn.commit();
    if (k)
        for (uint32_t b = 0; b < nseq; b++) {
            SeqHost &s = c->seqs[sid(ids, b)];
            s.stored_end = std::max(s.stored_end, s.pos + 1);
        }
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    if (int rc = sync_tables(c, st))
        return rc;
    const uint32_t *d_seq, *d_t;
    if (int rc = upload_rows(c, nseq, ids, nullptr, st, &d_seq, &d_t))
        return rc;
    AttnArgs a = attn_args(c, layer, nseq, q, gate, out, max_total, sum_total);
    a.row_seq = d_seq;
    a.row_t = d_t;
    a.k_new = k;
    a.v_new = v;
    if (psp.on) {
        a.chunk = psp.n_sh;
        a.max_chunks = psp.max_chunks;
        a.part = c->d_part;
        if (int rc = prefix_pass(c, a, nseq, ids, psp, st))
            return rc;
        a.chunk_lo = 1;
        return run_attend(c, a, st, c->d_part);
    }
    return run_attend(c, a, st);
}

int nda_decode(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
               const float *gate, float *out, void *stream)
{
    return decode_impl(c, layer, nseq, ids, q, nullptr, nullptr, gate, out, stream);
}

// nda_decode with its scratch in this device's static array instead of
// context buffers grown by hipMalloc: the ids are copied to the array's head
// and the split-KV partials follow at the next 256-byte boundary. Nothing in
// the array must start at zero: the merge reads only the partials the same
// call's attend launch writes. No profiling events are recorded.
int nda_decode_noalloc(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
                       const float *gate, float *out, void *stream)
{
    uint32_t max_total;
    uint64_t sum_total;
    if (int rc = decode_check(c, layer, nseq, ids, q, out, &max_total, &sum_total))
        return rc;
    if (!c->scratch)
        return fail(c, NDA_ERR_STATE, "nda_decode_noalloc: no scratch address for this device");
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    AttnArgs a = attn_args(c, layer, nseq, q, gate, out, max_total, sum_total);
    const uint64_t ids_bytes = ids ? (uint64_t)nseq * sizeof(uint32_t) : 0;
    const uint64_t part_off = (ids_bytes + 255) & ~(uint64_t)255;
    const bool split = a.max_chunks > 1 && !mfma_decode(c, a);
    const uint64_t part_bytes =
        split ? (uint64_t)a.rows * a.nh * a.max_chunks * (c->cfg.v_head_dim + 2) * sizeof(float) : 0;
    if (part_off + part_bytes > NDA_NOALLOC_SCRATCH_BYTES)
        return fail(c, NDA_ERR_RANGE,
                    "nda_decode_noalloc: %u sequence ids and %u-chunk split-KV partials need %llu bytes of "
                    "scratch, more than its %u",
                    ids ? nseq : 0u, a.max_chunks, (unsigned long long)(part_off + part_bytes),
                    (unsigned)NDA_NOALLOC_SCRATCH_BYTES);
    if (int rc = sync_tables(c, st))
        return rc;
    if (ids) {
        if (int rc = upload(c, c->scratch, ids, ids_bytes, st))
            return rc;
        a.row_seq = reinterpret_cast<const uint32_t *>(c->scratch);
    }
    return run_attend(c, a, st, split ? reinterpret_cast<float *>(c->scratch + part_off) : nullptr, false, false);
}

// Store, then attend. Small batches (launch latency dominates, e.g. one
// engine session) fuse both into one launch: the decode work-group owning
// the new slot quantises and stores it before attending. Large batches keep
// two launches: a store plus barrier at the head of every one of tens of
// thousands of work-groups costs more than the separate append kernel; GQA
// groups the MFMA decode serves switch to it (and so to two launches) from
// 4 work items per CU, and so do batches on one shared prefix that its
// decode pass serves.
int nda_step(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
             const float *k, const float *v, const float *gate, float *out, void *stream)
{
    if (c && nseq && (!k || !v))
        return fail(c, NDA_ERR_ARG, "null k/v");
    const uint64_t units = c ? (uint64_t)nseq * c->cfg.n_kv_heads : 0;
    int32_t pfx;
    uint32_t nsh;
    if (c && (units >= 16ull * (uint64_t)c->cus || (mfma_decode_geo(c) && units >= 4ull * (uint64_t)c->cus) ||
              (check_ids(c, nseq, ids) == NDA_OK && prefix_split_batch(c, nseq, ids, &pfx, &nsh)))) {
        // The decode's buffers first: once the append has stored this
        // position, a decode that fails for want of memory would leave the
        // step half done.
        if (layer < c->cfg.n_layers && check_ids(c, nseq, ids) == NDA_OK) {
            uint32_t max_total;
            uint64_t sum_total;
            decode_totals(c, nseq, ids, &max_total, &sum_total);
            PrefixSplit psp;
            if (int rc = decode_reserve(c, nseq, ids, false, max_total, sum_total, psp))
                return rc;
        }
        if (int rc = nda_kv_append(c, layer, nseq, ids, k, v, stream))
            return rc;
        return decode_impl(c, layer, nseq, ids, q, nullptr, nullptr, gate, out, stream);
    }
    return decode_impl(c, layer, nseq, ids, q, k, v, gate, out, stream);
}

// What a chunk must satisfy before nda_prefill changes anything: no ring
// wrap inside it, and an attached sequence positioned past its prefix.
static int prefill_check(nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens)
{
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t qq = sid(ids, b);
        const SeqHost &s = c->seqs[qq];
        if ((uint64_t)s.pos + n_tokens[b] > c->cfg.window)
            return fail(c, NDA_ERR_RANGE,
                        "sequence %u: prefill of %u tokens at position %u would wrap the ring (window %u)",
                        qq, n_tokens[b], s.pos, c->cfg.window);
        if (s.prefix >= 0 && s.pos < s.n_sink)
            return fail(c, NDA_ERR_STATE, "sequence %u positioned inside its shared prefix", qq);
    }
    return NDA_OK;
}

// What one nda_prefill call launches: rows, the visible runs they attend,
// the kernel (VALU or MFMA) and the MFMA work-group size and work list.
struct PrefillPlan {
    uint64_t rows = 0, sum_total = 0;
    uint32_t max_total = 0, rep = 1, trows = 0, nseq = 0;
    int waves = 4;
    bool valu = false;
    size_t n_items = 0;
};

// Work order of the MFMA prefill items. The kernel gives work-group w the
// item (w % 8) * (n / 8) + w / 8: XCD x (w % 8) runs the x-th eighth of the
// list, in order. The (sequence, kv-head) groups are sorted by the keys
// they visit (position plus chunk), most first, and dealt in turn to the
// eight ranges; each range is padded to the longest with empty items. A
// launch of ragged chunks (L ~ U[8K, 32K]) then ends on short items on
// every XCD, rather than on whichever long items came last. A group's row
// tiles stay adjacent in one range, where L2 serves their shared K/V.
static uint32_t prefill_bins(const nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens,
                             uint32_t rep, uint32_t trows, std::vector<std::pair<uint32_t, uint32_t>> (&bins)[8])
{
    std::vector<std::pair<uint64_t, uint32_t>> key;      // (keys visited, batch index)
    for (uint32_t b = 0; b < nseq; b++)
        if (n_tokens[b])
            key.push_back({(uint64_t)c->seqs[sid(ids, b)].pos + n_tokens[b], b});
    std::stable_sort(key.begin(), key.end(), [](const auto &x, const auto &y) { return x.first > y.first; });
    uint32_t load[8] = {}, rank = 0;
    for (auto &bin : bins)
        bin.clear();
    for (const auto &kb : key) {
        const uint32_t nt = (n_tokens[kb.second] * rep + trows - 1) / trows;
        for (uint32_t g = 0; g < c->cfg.n_kv_heads; g++, rank++) {
            bins[rank % 8].push_back({kb.second, g});
            load[rank % 8] += nt;
        }
    }
    return *std::max_element(load, load + 8);
}

static int prefill_plan(nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens, PrefillPlan &pl)
{
    pl = PrefillPlan();
    pl.nseq = nseq;
    for (uint32_t b = 0; b < nseq; b++) {
        const SeqHost &s = c->seqs[sid(ids, b)];
        if (n_tokens[b]) {
            const Vis v = visible(s, s.pos + n_tokens[b] - 1, c->cfg.window);
            pl.max_total = std::max(pl.max_total, v.n_sh + v.n_own);
            pl.sum_total += (uint64_t)n_tokens[b] * (v.n_sh + v.n_own);
        }
        pl.rows += n_tokens[b];
    }
    if (pl.rows > (1u << 26))
        return fail(c, NDA_ERR_ARG, "too many prefill tokens (%llu)", (unsigned long long)pl.rows);
    // The VALU kernel serves shapes the MFMA tiles are not built for (and
    // every shape when the config asks for it).
    pl.valu = (c->cfg.flags & NDA_FLAG_PREFILL_VALU) || !prefill_mfma_supported(c->geo);
    // MFMA work items = (batch index, kv-head, tile of 32*W query rows).
    // Work-group size by the longest chunk: 64-row groups for short
    // suffixes, 256-row groups (K/V staged once for 8 waves) for long ones.
    pl.rep = c->cfg.n_heads / c->cfg.n_kv_heads;
    uint32_t max_rows = 0;
    for (uint32_t b = 0; b < nseq; b++)
        max_rows = std::max(max_rows, n_tokens[b] * pl.rep);
    pl.waves = max_rows <= 64 ? 2 : (max_rows >= 256 ? 8 : 4);
    if (pl.waves == 8 && !(c->geo.kv_f16 && c->geo.rep == 1))
        pl.waves = 4;
#ifdef NDA_PF_FORCE_W     // build-time tuning knob: one work-group size for every chunk
    pl.waves = NDA_PF_FORCE_W;
#endif
    pl.trows = 32u * pl.waves;
    std::vector<std::pair<uint32_t, uint32_t>> bins[8];
    pl.n_items = 8 * (size_t)prefill_bins(c, nseq, ids, n_tokens, pl.rep, pl.trows, bins);
    return NDA_OK;
}

// The device buffers a planned prefill needs: row staging and either the
// partials of split VALU rows or the MFMA work list.
static int prefill_reserve(nda_ctx *c, const PrefillPlan &pl)
{
    if (pl.rows == 0)
        return NDA_OK;
    if (pl.valu)
        return reserve_attend(c, (uint32_t)pl.rows, true, pl.max_total, pl.sum_total);
    if (int rc = ensure_rows(c, pl.rows))
        return rc;
    return ensure_pf(c, 8 * pl.n_items);
}

int nda_prefill(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens,
                const float *q, const float *k, const float *v, const float *gate, float *out, void *stream)
{
    if (!c || (nseq && (!n_tokens || !q || !k || !v || !out)))
        return c ? fail(c, NDA_ERR_ARG, "null argument") : NDA_ERR_ARG;
    if (!aligned16(q) || !aligned16(out))
        return fail(c, NDA_ERR_ARG, "q and out must be 16-byte aligned");
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    if (int rc = prefill_check(c, nseq, ids, n_tokens))
        return rc;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    PrefillPlan pl;
    if (int rc = prefill_plan(c, nseq, ids, n_tokens, pl))
        return rc;
    if (pl.rows == 0)
        return NDA_OK;
    const uint64_t rows = pl.rows;
    const uint32_t max_total = pl.max_total, rep = pl.rep, trows = pl.trows;
    const uint64_t sum_total = pl.sum_total;
    const bool valu = pl.valu;
    const int waves = pl.waves;
    // Buffers first, then pages (given back if the pool runs out part-way):
    // a call that fails for want of memory changes nothing.
    if (int rc = prefill_reserve(c, pl))
        return rc;
    PageTxn txn(c->pt);
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t qq = sid(ids, b);
        if (n_tokens[b])
            if (int rc = back_positions(c, qq, c->seqs[qq].pos, n_tokens[b]))
                return rc;
    }
    txn.commit();
    for (uint32_t b = 0; b < nseq; b++) {
        SeqHost &s = c->seqs[sid(ids, b)];
        if (n_tokens[b])
            s.stored_end = std::max(s.stored_end, s.pos + n_tokens[b]);
    }
    std::vector<uint32_t> rseq(rows), rt(rows);
    for (uint32_t b = 0, r = 0; b < nseq; b++)
        for (uint32_t t = 0; t < n_tokens[b]; t++, r++) {
            rseq[r] = sid(ids, b);
            rt[r] = t;
        }
    if (int rc = sync_tables(c, st))
        return rc;
    const uint32_t *d_seq, *d_t;
    if (int rc = upload_rows(c, (uint32_t)rows, rseq.data(), rt.data(), st, &d_seq, &d_t))
        return rc;
    {
        AppendArgs a{};
        a.k = k;
        a.v = v;
        a.pool = c->pool + (uint64_t)layer * c->pg.layer_bytes;
        a.page_table = c->d_pages;
        a.seqs = c->d_seqs;
        a.row_seq = d_seq;
        a.row_t = d_t;
        a.pg = c->pg;
        a.rows = (uint32_t)rows;
        ProfScope ps(c, NDA_K_APPEND, st);
        hipError_t e = launch_append(c->geo, a, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "append kernel launch");
    }
    if (valu) {
        AttnArgs a = attn_args(c, layer, (uint32_t)rows, q, gate, out, max_total, sum_total);
        a.row_seq = d_seq;
        a.row_t = d_t;
        return run_attend(c, a, st);
    }
    // One record per work item with all a work-group needs to start (its
    // first reads then wait on one scalar load, not a chain of three):
    // sequence (~0: padding), kv-head, row tile, first packed token, tokens,
    // position, shared-prefix slots, prefix id (-1: none).
    // in the order of prefill_bins (the same as planned: positions have not
    // changed since)
    std::vector<uint32_t> tok0(nseq);
    for (uint32_t b = 0, tok = 0; b < nseq; b++) {
        tok0[b] = tok;
        tok += n_tokens[b];
    }
    std::vector<std::pair<uint32_t, uint32_t>> bins[8];
    const uint32_t per_bin = prefill_bins(c, nseq, ids, n_tokens, rep, trows, bins);
    std::vector<uint32_t> items;
    items.reserve(8 * 8 * (size_t)per_bin);
    // key tiles of the longest item (its work-group's tile table): the
    // shared prefix's, then the own slots up to the chunk's last token
    uint32_t tab_cap = 0;
    for (const auto &bin : bins) {
        uint32_t n = 0;
        for (const auto &bg : bin) {
            const uint32_t b = bg.first, qq = sid(ids, b);
            const SeqHost &s = c->seqs[qq];
            const Vis v = visible(s, s.pos, c->cfg.window);
            tab_cap = std::max<uint32_t>(tab_cap, (v.n_sh + 31) / 32 + (s.pos + n_tokens[b] - v.n_sh + 31) / 32);
            const uint32_t nt = (n_tokens[b] * rep + trows - 1) / trows;
            for (uint32_t t = 0; t < nt; t++, n++) {
                const uint32_t rec[8] = {qq, bg.second, t, tok0[b], n_tokens[b], s.pos, v.n_sh, (uint32_t)s.prefix};
                items.insert(items.end(), rec, rec + 8);
            }
        }
        for (; n < per_bin; n++) {
            const uint32_t pad[8] = {0xFFFFFFFFu, 0, 0, 0, 0, 0, 0, 0};
            items.insert(items.end(), pad, pad + 8);
        }
    }
    if (items.size() != 8 * pl.n_items)
        return fail(c, NDA_ERR_STATE, "prefill work list: size differs from its plan");
    if (int rc = upload(c, c->d_pf, items.data(), items.size() * 4, st))
        return rc;
    PrefillArgs pa{};
    pa.q = q;
    pa.gate = gate;
    pa.out = out;
    pa.pool = c->pool + (uint64_t)layer * c->pg.layer_bytes;
    pa.page_table = c->d_pages;
    pa.prefix_pages = c->d_prefix_pages;
    pa.seqs = c->d_seqs;
    pa.items = c->d_pf;
    pa.tab_cap = tab_cap;
    pa.pg = c->pg;
    pa.n_items = (uint32_t)(items.size() / 8);
    pa.nh = c->cfg.n_heads;
    pa.qscale = (float)(1.4426950408889634 / std::sqrt((double)c->cfg.qk_head_dim));
    ProfScope ps(c, NDA_K_PREFILL, st);
    hipError_t e = launch_prefill(c->geo, pa, waves, st);
    if (e != hipSuccess)
        return hip_fail(c, e, "prefill kernel launch");
    return NDA_OK;
}

// ------------------------------------------------------- attention front

int nda_front_init(nda_ctx *c, const nda_front_config *fc)
{
    if (!c || !fc)
        return NDA_ERR_ARG;
    if (c->taps)
        return fail(c, NDA_ERR_STATE, "attention front already initialised");
    if (fc->taps < 1 || fc->taps > 8)
        return fail(c, NDA_ERR_ARG, "taps %u outside 1..8", fc->taps);
    if (!(fc->rope_theta > 0.0f))
        return fail(c, NDA_ERR_ARG, "rope_theta must be positive");
    const nda_config &g = c->cfg;
    const uint32_t max_pos = fc->max_pos ? fc->max_pos : 65536u;
    if (max_pos > (1u << 24))
        return fail(c, NDA_ERR_ARG, "max_pos %u above 2^24 (positions must be exact in fp32)", max_pos);
    const uint32_t dcol = g.n_heads * g.qk_head_dim + g.n_kv_heads * (g.qk_head_dim + g.v_head_dim);
    const uint32_t half = g.qk_head_dim / 2;
    const uint64_t block = (uint64_t)g.n_layers * fc->taps * dcol;
    // Rotary table: the engine's inverse frequencies (nd_model.c:1233-1236)
    // and per-position cos/sin (:2949-2954), with the same libm calls.
    std::vector<float> inv(half);
    for (uint32_t i = 0; i < half; i++)
        inv[i] = 1.0f / powf(fc->rope_theta, (float)(2 * i) / (float)g.qk_head_dim);
    std::vector<float2> rope((size_t)max_pos * half);
    for (uint32_t p = 0; p < max_pos; p++)
        for (uint32_t i = 0; i < half; i++) {
            const float angle = (float)p * inv[i];
            rope[(size_t)p * half + i] = make_float2(cosf(angle), sinf(angle));
        }
    // All six buffers or none: a failed allocation frees the ones made here.
    const size_t hist_bytes = block * sizeof(float);
    struct {
        void **ptr;
        size_t bytes;
    } bufs[] = {{(void **)&c->d_hist, hist_bytes * g.max_seqs},
                {(void **)&c->d_snap_hist, hist_bytes * g.max_seqs},
                {(void **)&c->d_prefix_hist, hist_bytes * std::max(1u, g.max_prefixes)},
                {(void **)&c->d_front_w, (size_t)g.n_layers * fc->taps * dcol * sizeof(float)},
                {(void **)&c->d_front_norm, (size_t)g.n_layers * 2 * g.qk_head_dim * sizeof(float)},
                {(void **)&c->d_rope, rope.size() * sizeof(float2)}};
    for (auto &b : bufs) {
        *b.ptr = dev_alloc(b.bytes);
        if (!*b.ptr) {
            for (auto &u : bufs) {
                dev_free(*u.ptr);
                *u.ptr = nullptr;
            }
            return fail(c, NDA_ERR_NOMEM, "device allocation of %zu bytes failed", b.bytes);
        }
    }
    for (auto &b : bufs)
        c->dev_bytes += b.bytes;
    HIPC(c, hipMemset(c->d_hist, 0, hist_bytes * g.max_seqs));
    HIPC(c, hipMemset(c->d_snap_hist, 0, hist_bytes * g.max_seqs));
    HIPC(c, hipMemcpy(c->d_rope, rope.data(), rope.size() * sizeof(float2), hipMemcpyHostToDevice));
    c->taps = fc->taps;
    c->max_pos = max_pos;
    c->dcol = dcol;
    c->hist_block = block;
    c->front_w_set.assign(g.n_layers, 0);
    return NDA_OK;
}

int nda_front_weights(nda_ctx *c, uint32_t layer, const float *tap_q, const float *tap_k,
                      const float *tap_v, const float *norm_q, const float *norm_k)
{
    if (!c)
        return NDA_ERR_ARG;
    if (!c->taps)
        return fail(c, NDA_ERR_STATE, "attention front not initialised (nda_front_init)");
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (!tap_q || !tap_k || !tap_v || !norm_q || !norm_k)
        return fail(c, NDA_ERR_ARG, "null weight array");
    const nda_config &g = c->cfg;
    const uint32_t dq = g.n_heads * g.qk_head_dim, dk = g.n_kv_heads * g.qk_head_dim,
                   dv = g.n_kv_heads * g.v_head_dim;
    // Device rows are [tap][q | k | v] so one tap's weights for a column sit
    // at the column's offset in every row.
    std::vector<float> w((size_t)c->taps * c->dcol);
    for (uint32_t j = 0; j < c->taps; j++) {
        float *r = &w[(size_t)j * c->dcol];
        std::memcpy(r, tap_q + (size_t)j * dq, dq * sizeof(float));
        std::memcpy(r + dq, tap_k + (size_t)j * dk, dk * sizeof(float));
        std::memcpy(r + dq + dk, tap_v + (size_t)j * dv, dv * sizeof(float));
    }
    std::vector<float> nrm(2 * (size_t)g.qk_head_dim);
    std::memcpy(nrm.data(), norm_q, g.qk_head_dim * sizeof(float));
    std::memcpy(nrm.data() + g.qk_head_dim, norm_k, g.qk_head_dim * sizeof(float));
    HIPC(c, hipMemcpy(c->d_front_w + (size_t)layer * c->taps * c->dcol, w.data(), w.size() * sizeof(float),
                      hipMemcpyHostToDevice));
    HIPC(c, hipMemcpy(c->d_front_norm + (size_t)layer * 2 * g.qk_head_dim, nrm.data(),
                      nrm.size() * sizeof(float), hipMemcpyHostToDevice));
    c->front_w_set[layer] = 1;
    return NDA_OK;
}

namespace {

// Checks shared by the front entry points: initialised, weights present,
// each sequence at most once, every position inside the rotary table.
int front_check(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens)
{
    if (!c->taps)
        return fail(c, NDA_ERR_STATE, "attention front not initialised (nda_front_init)");
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (!c->front_w_set[layer])
        return fail(c, NDA_ERR_STATE, "no front weights for layer %u (nda_front_weights)", layer);
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    c->seen.assign(c->cfg.max_seqs, 0);
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t q = sid(ids, b);
        if (c->seen[q]++)
            return fail(c, NDA_ERR_ARG, "sequence %u listed twice", q);
        const uint32_t n = n_tokens ? n_tokens[b] : 1u;
        if (n && (uint64_t)c->seqs[q].pos + n > c->max_pos)
            return fail(c, NDA_ERR_RANGE, "sequence %u: position %u beyond the rotary table (max_pos %u)", q,
                        c->seqs[q].pos + n - 1, c->max_pos);
    }
    return NDA_OK;
}

FrontArgs front_args(nda_ctx *c, uint32_t layer)
{
    FrontArgs a{};
    a.hist = c->d_hist;
    a.w = c->d_front_w + (size_t)layer * c->taps * c->dcol;
    a.norm = c->d_front_norm + (size_t)layer * 2 * c->cfg.qk_head_dim;
    a.rope = c->d_rope;
    a.seqs = c->d_seqs;
    a.pg = c->pg;
    a.layer = layer;
    a.n_layers = c->cfg.n_layers;
    a.taps = c->taps;
    a.nh = c->cfg.n_heads;
    a.nkv = c->cfg.n_kv_heads;
    a.qk = c->cfg.qk_head_dim;
    a.vd = c->cfg.v_head_dim;
    return a;
}

} // namespace

int nda_front(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens,
              const float *q, const float *k, const float *v, float *q_out, float *k_out, float *v_out,
              void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (nseq && (!q || !k || !v || !q_out || !k_out || !v_out))
        return fail(c, NDA_ERR_ARG, "null q/k/v or output");
    if (int rc = front_check(c, layer, nseq, ids, n_tokens))
        return rc;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(k_out) || !aligned16(v_out))
        return fail(c, NDA_ERR_ARG, "q/k/v and k_out/v_out must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    uint64_t rows = 0;
    bool multi = false;
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t n = n_tokens ? n_tokens[b] : 1u;
        rows += n;
        multi |= n > 1;
    }
    if (rows == 0)
        return NDA_OK;
    if (rows > (1u << 26))
        return fail(c, NDA_ERR_ARG, "too many front rows (%llu)", (unsigned long long)rows);
    if (int rc = sync_tables(c, st))
        return rc;
    if (int rc = hist_flush(c, st))
        return rc;
    if (int rc = ensure_buf(c, c->d_front_rows, c->front_rows_cap, 3 * rows))
        return rc;
    std::vector<uint32_t> host(3 * rows);
    for (uint32_t b = 0, r = 0; b < nseq; b++) {
        const uint32_t n = n_tokens ? n_tokens[b] : 1u;
        for (uint32_t t = 0; t < n; t++, r++) {
            host[r] = sid(ids, b);
            host[rows + r] = t;
            host[2 * rows + r] = n;
        }
    }
    if (int rc = upload(c, c->d_front_rows, host.data(), host.size() * 4, st))
        return rc;
    FrontArgs a = front_args(c, layer);
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_out = v_out;
    a.row_seq = c->d_front_rows;
    a.row_t = c->d_front_rows + rows;
    a.rows = (uint32_t)rows;
    a.hist_write = multi ? 0u : 1u;
    {
        ProfScope ps(c, NDA_K_FRONT, st);
        hipError_t e = launch_front(c->geo, a, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "front kernel launch");
    }
    if (multi) {
        HistTailArgs h{};
        h.q = q;
        h.k = k;
        h.v = v;
        h.hist = c->d_hist;
        h.seqs = c->d_seqs;
        h.row_seq = a.row_seq;
        h.row_t = a.row_t;
        h.row_n = c->d_front_rows + 2 * rows;
        h.rows = (uint32_t)rows;
        h.layer = layer;
        h.n_layers = c->cfg.n_layers;
        h.taps = c->taps;
        h.dq = c->cfg.n_heads * c->cfg.qk_head_dim;
        h.dk = c->cfg.n_kv_heads * c->cfg.qk_head_dim;
        h.dv = c->cfg.n_kv_heads * c->cfg.v_head_dim;
        hipError_t e = launch_hist_tail(h, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "history write-back launch");
    }
    return NDA_OK;
}

int nda_attention(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
                  const float *k, const float *v, const float *gate, float *out, void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (nseq && (!q || !k || !v || !out))
        return fail(c, NDA_ERR_ARG, "null q/k/v/out");
    if (int rc = front_check(c, layer, nseq, ids, nullptr))
        return rc;
    if (nseq == 0)
        return NDA_OK;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v))
        return fail(c, NDA_ERR_ARG, "q/k/v must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    // Buffers first (the front's q, the row staging, the decode's partials),
    // then pages: a call that fails for want of memory changes nothing.
    const size_t dq = (size_t)c->cfg.n_heads * c->cfg.qk_head_dim;
    if (int rc = ensure_buf(c, c->d_qfront, c->qfront_cap, (size_t)nseq * dq))
        return rc;
    if (int rc = hist_reserve(c, 0))
        return rc;
    PageTxn txn(c->pt);
    uint32_t max_total = 0;
    uint64_t sum_total = 0;
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t qq = sid(ids, b);
        if (int rc = back_positions(c, qq, c->seqs[qq].pos, 1))
            return rc;
        const Vis vv = visible(c->seqs[qq], c->seqs[qq].pos, c->cfg.window);
        max_total = std::max(max_total, vv.n_sh + vv.n_own);
        sum_total += vv.n_sh + vv.n_own;
    }
    if (int rc = reserve_attend(c, nseq, ids != nullptr, max_total, sum_total))
        return rc;
    txn.commit();
    for (uint32_t b = 0; b < nseq; b++) {
        SeqHost &s = c->seqs[sid(ids, b)];
        s.stored_end = std::max(s.stored_end, s.pos + 1);
    }
    if (int rc = sync_tables(c, st))
        return rc;
    if (int rc = hist_flush(c, st))
        return rc;
    const uint32_t *d_seq, *d_t;
    if (int rc = upload_rows(c, nseq, ids, nullptr, st, &d_seq, &d_t))
        return rc;
    FrontArgs a = front_args(c, layer);
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_out = c->d_qfront;
    a.row_seq = d_seq;
    a.rows = nseq;
    a.hist_write = 1;
    a.pool = c->pool + (uint64_t)layer * c->pg.layer_bytes;
    a.page_table = c->d_pages;
    {
        ProfScope ps(c, NDA_K_FRONT, st);
        hipError_t e = launch_front(c->geo, a, st);
        if (e != hipSuccess)
            return hip_fail(c, e, "front kernel launch");
    }
    return decode_impl(c, layer, nseq, ids, c->d_qfront, nullptr, nullptr, gate, out, stream);
}

int nda_front_hist(nda_ctx *c, uint32_t seq, int snap, float *dst, void *stream)
{
    if (!c || !dst)
        return c ? fail(c, NDA_ERR_ARG, "null destination") : NDA_ERR_ARG;
    if (!c->taps)
        return fail(c, NDA_ERR_STATE, "attention front not initialised (nda_front_init)");
    if (int rc = check_seq(c, seq))
        return rc;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    if (int rc = hist_flush(c, st))
        return rc;
    const float *src = snap ? hist_snap(c, seq) : hist_live(c, seq);
    HIPC(c, hipMemcpyAsync(dst, src, c->hist_block * sizeof(float), hipMemcpyDeviceToHost, st));
    HIPC(c, hipStreamSynchronize(st));
    return NDA_OK;
}

int nda_sync(nda_ctx *c, void *stream)
{
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess)
        return hip_fail(c, e, "hipStreamSynchronize");
    // the context's work on that stream is done: the next call, on any
    // stream, waits for nothing (and the stream may be destroyed)
    if (c && c->has_stream && c->last_stream == (hipStream_t)stream)
        c->has_stream = false;
    return NDA_OK;
}

// Page and in-page slot of `count` positions from p0 of one sequence.
static int locate(nda_ctx *c, uint32_t seq, uint32_t p0, uint32_t count, bool for_write,
                  std::vector<int32_t> &pg, std::vector<uint32_t> &off)
{
    SeqHost &s = c->seqs[seq];
    pg.resize(count);
    off.resize(count);
    const uint32_t P = c->cfg.page_size;
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t p = p0 + i;
        if (s.prefix >= 0 && p < s.n_sink) {
            if (for_write)
                return fail(c, NDA_ERR_STATE, "position %u belongs to the shared prefix", p);
            pg[i] = c->pt.prefix_pages[(size_t)s.prefix * c->pg.pages_per_seq + p / P];
            off[i] = p % P;
            continue;
        }
        if (!for_write) {
            // readable iff stored and not yet overwritten by the ring
            const uint32_t rcap = c->cfg.window - s.n_sink;
            if (p >= s.stored_end)
                return fail(c, NDA_ERR_RANGE, "position %u was never stored", p);
            if (p >= s.n_sink && (s.stored_end - p > rcap || p < s.ring_lo))
                return fail(c, NDA_ERR_RANGE, "position %u has left the ring", p);
        }
        const uint32_t sl = own_slot(s, p, c->cfg.window);
        if (for_write)
            if (int rc = back_slots(c, seq, sl, sl + 1))
                return rc;
        pg[i] = c->pt.pages[(size_t)seq * c->pg.pages_per_seq + sl / P];
        off[i] = sl % P;
        if (pg[i] < 0)
            return fail(c, NDA_ERR_STATE, "position %u was never stored", p);
    }
    return NDA_OK;
}

static int kv_stage(nda_ctx *c, uint32_t layer, uint32_t seq, uint32_t p0, uint32_t count, void *k, void *v,
                    float *ks, float *vs, bool write)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_seq(c, seq))
        return rc;
    if (layer >= c->cfg.n_layers || !k || !v)
        return fail(c, NDA_ERR_ARG, "bad layer or null buffer");
    if (count == 0)
        return NDA_OK;
    if (write && c->cfg.kv_dtype == NDA_KV_INT8 && (!ks || !vs))
        return fail(c, NDA_ERR_ARG, "int8 write needs scales");
    const size_t es = c->cfg.kv_dtype == NDA_KV_F16 ? 2 : 1;
    const size_t nkv = c->cfg.n_kv_heads;
    const size_t kb = count * nkv * c->cfg.qk_head_dim * es, vb = count * nkv * c->cfg.v_head_dim * es;
    const size_t sb = count * nkv * sizeof(float);
    const size_t ib = count * (sizeof(int32_t) + sizeof(uint32_t));
    const size_t total = kb + vb + 2 * sb + ib + 64;
    if (int rc = ensure_stage(c, total))
        return rc;
    std::vector<int32_t> pg;
    std::vector<uint32_t> off;
    PageTxn txn(c->pt);
    if (int rc = locate(c, seq, p0, count, write, pg, off))
        return rc;
    txn.commit();
    uint8_t *d = c->d_stage;
    StageArgs a{};
    a.pool = c->pool + (uint64_t)layer * c->pg.layer_bytes;
    a.stage_ks = reinterpret_cast<float *>(d);
    a.stage_vs = reinterpret_cast<float *>(d + sb);
    a.pages_for_slot = reinterpret_cast<int32_t *>(d + 2 * sb);
    a.slot_in_page = reinterpret_cast<uint32_t *>(d + 2 * sb + count * 4);
    a.stage_k = d + 2 * sb + count * 8;
    a.stage_v = a.stage_k + kb;
    a.count = count;
    a.pg = c->pg;
    if (int rc = on_stream(c, nullptr))
        return rc;
    if (int rc = sync_tables(c, nullptr))
        return rc;
    HIPC(c, hipMemcpy((void *)a.pages_for_slot, pg.data(), count * 4, hipMemcpyHostToDevice));
    HIPC(c, hipMemcpy((void *)a.slot_in_page, off.data(), count * 4, hipMemcpyHostToDevice));
    if (write) {
        HIPC(c, hipMemcpy(a.stage_k, k, kb, hipMemcpyHostToDevice));
        HIPC(c, hipMemcpy(a.stage_v, v, vb, hipMemcpyHostToDevice));
        if (c->cfg.kv_dtype == NDA_KV_INT8) {
            HIPC(c, hipMemcpy(a.stage_ks, ks, sb, hipMemcpyHostToDevice));
            HIPC(c, hipMemcpy(a.stage_vs, vs, sb, hipMemcpyHostToDevice));
        }
        hipError_t e = launch_scatter(c->geo, a, nullptr);
        if (e != hipSuccess)
            return hip_fail(c, e, "scatter");
        HIPC(c, hipDeviceSynchronize());
        SeqHost &sw = c->seqs[seq];
        sw.stored_end = std::max(sw.stored_end, p0 + count);
    } else {
        hipError_t e = launch_gather(c->geo, a, nullptr);
        if (e != hipSuccess)
            return hip_fail(c, e, "gather");
        HIPC(c, hipDeviceSynchronize());
        HIPC(c, hipMemcpy(k, a.stage_k, kb, hipMemcpyDeviceToHost));
        HIPC(c, hipMemcpy(v, a.stage_v, vb, hipMemcpyDeviceToHost));
        if (ks)
            HIPC(c, hipMemcpy(ks, a.stage_ks, sb, hipMemcpyDeviceToHost));
        if (vs)
            HIPC(c, hipMemcpy(vs, a.stage_vs, sb, hipMemcpyDeviceToHost));
    }
    return NDA_OK;
}

int nda_kv_read(nda_ctx *c, uint32_t layer, uint32_t seq, uint32_t p0, uint32_t count, void *k, void *v,
                float *ks, float *vs)
{
    return kv_stage(c, layer, seq, p0, count, k, v, ks, vs, false);
}

int nda_kv_write(nda_ctx *c, uint32_t layer, uint32_t seq, uint32_t p0, uint32_t count, const void *k,
                 const void *v, const float *ks, const float *vs)
{
    return kv_stage(c, layer, seq, p0, count, const_cast<void *>(k), const_cast<void *>(v),
                    const_cast<float *>(ks), const_cast<float *>(vs), true);
}

int nda_kv_fill_normal(nda_ctx *c, uint32_t nseq, const uint32_t *ids, uint64_t seed, void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    if (ids)
        if (int rc = ensure_rows(c, nseq))
            return rc;
    PageTxn txn(c->pt);
    for (uint32_t b = 0; b < nseq; b++) {
        const uint32_t qq = sid(ids, b);
        const SeqHost &s = c->seqs[qq];
        if (s.pos == 0)
            continue;
        const Vis v = visible(s, s.pos - 1, c->cfg.window);
        if (int rc = back_slots(c, qq, 0, v.n_own))
            return rc;
    }
    txn.commit();
    for (uint32_t b = 0; b < nseq; b++) {
        SeqHost &s = c->seqs[sid(ids, b)];
        s.stored_end = std::max(s.stored_end, s.pos);
    }
    if (int rc = sync_tables(c, st))
        return rc;
    const uint32_t *d_seq, *d_t;
    if (int rc = upload_rows(c, nseq, ids, nullptr, st, &d_seq, &d_t))
        return rc;
    FillKvArgs a{};
    a.pool = c->pool;
    a.page_table = c->d_pages;
    a.prefix_pages = c->d_prefix_pages;
    a.seqs = c->d_seqs;
    a.seq_list = d_seq;
    a.nseq = nseq;
    a.n_layers = c->cfg.n_layers;
    a.seed = seed;
    a.pg = c->pg;
    hipError_t e = launch_fill_kv(c->geo, a, st);
    if (e != hipSuccess)
        return hip_fail(c, e, "fill kernel launch");
    return NDA_OK;
}

int nda_dev_alloc(void **ptr, size_t bytes)
{
    if (!ptr)
        return NDA_ERR_ARG;
    *ptr = dev_alloc(bytes);
    return *ptr ? NDA_OK : NDA_ERR_NOMEM;
}

int nda_dev_free(void *ptr)
{
    dev_free(ptr);
    return NDA_OK;
}

int nda_set_allocator(nda_alloc_fn alloc, nda_free_fn free_fn, void *user)
{
    if (!alloc != !free_fn)
        return NDA_ERR_ARG;
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    g_alloc = alloc ? alloc : default_alloc;
    g_free = alloc ? free_fn : default_free;
    g_alloc_user = alloc ? user : nullptr;
    return NDA_OK;
}

int nda_h2d(void *dst, const void *src, size_t bytes)
{
    return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_d2h(void *dst, const void *src, size_t bytes)
{
    return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

// ------------------------------------------------------- CQ projections

struct nda_cq {
    uint32_t out, in, in_pad, group, ngroup, bits, rowbytes;
    uint8_t *packed = nullptr;     // [out][rowbytes]
    uint16_t *norms = nullptr;     // [out][ngroup], 2-byte aligned copy
    float *cb = nullptr;           // [1 << bits]
    // split GEMM decode data (2-bit tensors, group >= 32)
    uint32_t *cw = nullptr;
    uint4 *tab = nullptr;
    int32_t *cexp = nullptr;
};

int nda_cq_create(uint32_t out, uint32_t in, uint32_t group, uint32_t bits, const void *blob,
                  const float *codebook, nda_cq **tp)
{
    if (!tp || !blob || !codebook || out == 0 || in == 0)
        return NDA_ERR_ARG;
    *tp = nullptr;
    if (bits < 2 || bits > 4 || group < 16 || group > 4096 || (group & (group - 1)))
        return NDA_ERR_UNSUPPORTED;
    nda_cq *t = new (std::nothrow) nda_cq();
    if (!t)
        return NDA_ERR_NOMEM;
    t->out = out;
    t->in = in;
    t->group = group;
    t->bits = bits;
    t->in_pad = (in + group - 1) / group * group;
    t->ngroup = t->in_pad / group;
    t->rowbytes = t->in_pad * bits / 8;
    if (t->in_pad > 16384) {
        delete t;
        return NDA_ERR_UNSUPPORTED;
    }
    const size_t pb = (size_t)out * t->rowbytes, nb = (size_t)out * t->ngroup * 2;
    // +4 bytes: the bitstream reader may touch the byte after a straddling field
    t->packed = static_cast<uint8_t *>(dev_alloc(pb + 4));
    t->norms = static_cast<uint16_t *>(dev_alloc(nb));
    t->cb = static_cast<float *>(dev_alloc(sizeof(float) << bits));
    if (!t->packed || !t->norms || !t->cb) {
        nda_cq_destroy(t);
        return NDA_ERR_NOMEM;
    }
    if (hipMemcpy(t->packed, blob, pb, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(t->packed + pb, 0, 4) != hipSuccess ||
        hipMemcpy(t->norms, (const uint8_t *)blob + pb, nb, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(t->cb, codebook, sizeof(float) << bits, hipMemcpyHostToDevice) != hipSuccess) {
        nda_cq_destroy(t);
        return NDA_ERR_HIP;
    }
    if (bits == 2 && group >= 32) {
        CqTabArgs ta{};
        ta.packed = t->packed;
        ta.norms = t->norms;
        ta.cb = t->cb;
        ta.out = out;
        ta.in_pad = t->in_pad;
        ta.ngroup = t->ngroup;
        ta.rowbytes = t->rowbytes;
        t->cw = static_cast<uint32_t *>(dev_alloc((size_t)t->in_pad / 32 * out * 8));
        t->tab = static_cast<uint4 *>(dev_alloc((size_t)t->ngroup * out * 16));
        t->cexp = static_cast<int32_t *>(dev_alloc((size_t)out * 4));
        if (!t->cw || !t->tab || !t->cexp) {
            nda_cq_destroy(t);
            return NDA_ERR_NOMEM;
        }
        ta.cw = t->cw;
        ta.tab = t->tab;
        ta.cexp = t->cexp;
        if (launch_cq_split_tables(ta, nullptr) != hipSuccess || hipStreamSynchronize(nullptr) != hipSuccess) {
            nda_cq_destroy(t);
            return NDA_ERR_HIP;
        }
    }
    *tp = t;
    return NDA_OK;
}

int nda_cq_destroy(nda_cq *t)
{
    if (!t)
        return NDA_OK;
    for (void *b : {(void *)t->packed, (void *)t->norms, (void *)t->cb, (void *)t->cw, (void *)t->tab,
                    (void *)t->cexp})
        dev_free(b);
    delete t;
    return NDA_OK;
}

uint32_t nda_cq_in_pad(const nda_cq *t) { return t ? t->in_pad : 0; }

int nda_cq_prepare(const nda_cq *t, uint32_t rows, const float *x, float *xh, void *stream)
{
    if (!t || (rows && (!x || !xh)))
        return NDA_ERR_ARG;
    if (((uintptr_t)x & 15) || ((uintptr_t)xh & 15))
        return NDA_ERR_ARG;
    CqPrepArgs a{};
    a.x = x;
    a.xh = xh;
    a.rows = rows;
    a.in = t->in;
    a.in_pad = t->in_pad;
    a.group = t->group;
    a.scale = 1.0f / sqrtf((float)t->group);      // nd_cq_prepare's scale
    return launch_cq_prepare(a, (hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_cq_gemm_many(const nda_cq *const *ts, uint32_t n, uint32_t rows, const float *xh, float *const *ys,
                     void *stream)
{
    if (!ts || !ys || n == 0 || n > (uint32_t)CQ_MAX_T || (rows && !xh))
        return NDA_ERR_ARG;
    if ((uintptr_t)xh & 15)
        return NDA_ERR_ARG;
    if ((uint64_t)rows > 0x7FFFFFFFull)
        return NDA_ERR_ARG;
    const nda_cq *t0 = ts[0];
    if (!t0)
        return NDA_ERR_ARG;
    CqGemmArgs a{};
    a.xh = xh;
    a.rows = rows;
    a.in_pad = t0->in_pad;
    a.group = t0->group;
    a.ngroup = t0->ngroup;
    a.bits = t0->bits;
    a.rowbytes = t0->rowbytes;
    a.nt = n;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < n; i++) {
        const nda_cq *t = ts[i];
        if (!t || (rows && !ys[i]))
            return NDA_ERR_ARG;
        if (t->in != t0->in || t->group != t0->group || t->bits != t0->bits)
            return NDA_ERR_ARG;     // one prepared activation serves them all
        a.y[i] = ys[i];
        a.packed[i] = t->packed;
        a.norms[i] = t->norms;
        a.cb[i] = t->cb;
        a.out[i] = t->out;
        a.tile0[i] = tiles;
        tiles += (t->out + 63) / 64;
    }
    a.tile0[n] = tiles;
    if (tiles > 65535)
        return NDA_ERR_ARG;
    return launch_cq_gemm(a, (hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_cq_gemm(const nda_cq *t, uint32_t rows, const float *xh, float *y, void *stream)
{
    return nda_cq_gemm_many(&t, 1, rows, xh, &y, stream);
}

static bool cq_split_ok(const nda_cq *t) { return t->bits == 2 && t->group >= 32; }
static bool cq_lut2_ok(const nda_cq *t) { return t->bits == 2 && t->in_pad <= (uint32_t)CQ_LUT_MAX_IN; }

int nda_cq_gemv_lut2(const nda_cq *const *ts, uint32_t n, uint32_t rows, const float *xh, float *const *ys,
                     void *stream)
{
    if (!ts || !ys || n == 0 || n > (uint32_t)CQ_MAX_T || (rows && !xh) || ((uintptr_t)xh & 15))
        return NDA_ERR_ARG;
    const nda_cq *t0 = ts[0];
    if (!t0)
        return NDA_ERR_ARG;
    if (rows > 65535)
        return NDA_ERR_UNSUPPORTED;
    CqGemmArgs a{};
    a.xh = xh;
    a.rows = rows;
    a.in_pad = t0->in_pad;
    a.group = t0->group;
    a.ngroup = t0->ngroup;
    a.bits = t0->bits;
    a.rowbytes = t0->rowbytes;
    a.nt = n;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < n; i++) {
        const nda_cq *t = ts[i];
        if (!t || (rows && !ys[i]))
            return NDA_ERR_ARG;
        if (t->in != t0->in || t->group != t0->group || t->bits != t0->bits)
            return NDA_ERR_ARG;     // one prepared activation serves them all
        if (!cq_lut2_ok(t))
            return NDA_ERR_UNSUPPORTED;
        a.y[i] = ys[i];
        a.packed[i] = t->packed;
        a.norms[i] = t->norms;
        a.cb[i] = t->cb;
        a.out[i] = t->out;
        a.tile0[i] = tiles;
        tiles += (t->out + CQ_LUT_OT - 1) / CQ_LUT_OT;
    }
    a.tile0[n] = tiles;
    return launch_cq_lut2(a, (hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

// rows rounded up to a block of 32: operand blocks (4 bytes per element), then the exponents
static size_t split_rows(uint32_t rows) { return ((size_t)rows + 31) & ~(size_t)31; }

size_t nda_cq_split_bytes(const nda_cq *t, uint32_t rows)
{
    return t ? split_rows(rows) * t->in_pad * 4 + (size_t)rows * 4 : 0;
}

int nda_cq_prepare_split(const nda_cq *t, uint32_t rows, const float *x, void *xs, void *stream)
{
    if (!t || (rows && (!x || !xs)))
        return NDA_ERR_ARG;
    if (((uintptr_t)x & 15) || ((uintptr_t)xs & 15))
        return NDA_ERR_ARG;
    if (t->group < 32)
        return NDA_ERR_UNSUPPORTED;
    CqPrepSplitArgs a{};
    a.x = x;
    a.xs = (_Float16 *)xs;
    a.rexp = (int32_t *)(a.xs + split_rows(rows) * t->in_pad * 2);
    a.rows = rows;
    a.in = t->in;
    a.in_pad = t->in_pad;
    a.group = t->group;
    a.scale = 1.0f / sqrtf((float)t->group);
    return launch_cq_prepare_split(a, (hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_cq_gemm_split_many(const nda_cq *const *ts, uint32_t n, uint32_t rows, const void *xs, float *const *ys,
                           void *stream)
{
    if (!ts || !ys || n == 0 || n > (uint32_t)CQ_MAX_T || (rows && !xs))
        return NDA_ERR_ARG;
    if (((uintptr_t)xs & 15) || (uint64_t)rows > 0x7FFFFFFFull)
        return NDA_ERR_ARG;
    const nda_cq *t0 = ts[0];
    if (!t0)
        return NDA_ERR_ARG;
    CqSplitArgs a{};
    a.xs = (const _Float16 *)xs;
    a.rexp = (const int32_t *)(a.xs + split_rows(rows) * t0->in_pad * 2);
    a.rows = rows;
    a.in_pad = t0->in_pad;
    a.log2_group = (uint32_t)__builtin_ctz(t0->group);
    a.nt = n;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < n; i++) {
        const nda_cq *t = ts[i];
        if (!t || (rows && !ys[i]))
            return NDA_ERR_ARG;
        if (t->in != t0->in || t->group != t0->group || t->bits != t0->bits)
            return NDA_ERR_ARG;
        if (!cq_split_ok(t))
            return NDA_ERR_UNSUPPORTED;
        a.y[i] = ys[i];
        a.cw[i] = t->cw;
        a.tab[i] = t->tab;
        a.cexp[i] = t->cexp;
        a.out[i] = t->out;
        a.tile0[i] = tiles;
        tiles += (t->out + CQ_SPLIT_NT - 1) / CQ_SPLIT_NT;
    }
    a.tile0[n] = tiles;
    if (tiles > 65535)
        return NDA_ERR_ARG;
    return launch_cq_gemm_split(a, (hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_cq_gemm_split(const nda_cq *t, uint32_t rows, const void *xs, float *y, void *stream)
{
    return nda_cq_gemm_split_many(&t, 1, rows, xs, &y, stream);
}

// n tensors sharing one input (q/k/v/gate, or out_proj alone) for the block
// paths: the engine's own LUT order for up to CQ_LUT_ROWS rows (bit-identical
// projections, so the front and the int8 store see the engine's values), the
// split-precision GEMM above that where every tensor allows it, the fp32 GEMM
// otherwise. xs holds nda_cq_split_bytes(ts[0], rows), at least the fp32
// prepared form's rows * in_pad floats.
constexpr uint32_t CQ_LUT_ROWS = 64;
static int cq_project(const nda_cq *const *ts, uint32_t n, uint32_t rows, const float *x, void *xs,
                      float *const *ys, hipStream_t st)
{
    bool split = true, lut = rows <= CQ_LUT_ROWS;
    for (uint32_t i = 0; i < n; i++) {
        split = split && cq_split_ok(ts[i]);
        lut = lut && cq_lut2_ok(ts[i]);
    }
    if (lut) {
        if (int rc = nda_cq_prepare(ts[0], rows, x, (float *)xs, st))
            return rc;
        return nda_cq_gemv_lut2(ts, n, rows, (const float *)xs, ys, st);
    }
    if (split) {
        if (int rc = nda_cq_prepare_split(ts[0], rows, x, xs, st))
            return rc;
        return nda_cq_gemm_split_many(ts, n, rows, xs, ys, st);
    }
    if (int rc = nda_cq_prepare(ts[0], rows, x, (float *)xs, st))
        return rc;
    return nda_cq_gemm_many(ts, n, rows, (const float *)xs, ys, st);
}

int nda_block_weights(nda_ctx *c, uint32_t layer, const nda_cq *q, const nda_cq *k, const nda_cq *v,
                      const nda_cq *gate, const nda_cq *out_proj)
{
    if (!c)
        return NDA_ERR_ARG;
    if (layer >= c->cfg.n_layers)
        return fail(c, NDA_ERR_ARG, "layer %u out of range", layer);
    if (!q || !k || !v || !gate || !out_proj)
        return fail(c, NDA_ERR_ARG, "null tensor");
    const nda_config &g = c->cfg;
    const uint32_t dq = g.n_heads * g.qk_head_dim, dk = g.n_kv_heads * g.qk_head_dim,
                   dv = g.n_kv_heads * g.v_head_dim, da = g.n_heads * g.v_head_dim;
    if (q->out != dq || k->out != dk || v->out != dv || gate->out != da || out_proj->in != da)
        return fail(c, NDA_ERR_ARG, "projection shapes do not match the attention geometry");
    const uint32_t dm = q->in;
    for (const nda_cq *t : {k, v, gate})
        if (t->in != dm || t->group != q->group || t->bits != q->bits)
            return fail(c, NDA_ERR_ARG, "q/k/v/gate must share d_model, group and width");
    if (out_proj->out != dm)
        return fail(c, NDA_ERR_ARG, "out_proj must map back to d_model (%u)", dm);
    if (c->d_model && c->d_model != dm)
        return fail(c, NDA_ERR_ARG, "d_model %u differs from an earlier layer's %u", dm, c->d_model);
    if (c->blk.empty())
        c->blk.assign(g.n_layers, {nullptr, nullptr, nullptr, nullptr, nullptr});
    c->d_model = dm;
    c->blk[layer] = {q, k, v, gate, out_proj};
    return NDA_OK;
}

int nda_attention_block(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *x,
                        float *out, void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (layer >= c->cfg.n_layers || c->blk.empty() || !c->blk[layer][0])
        return fail(c, NDA_ERR_STATE, "no projection weights for layer %u (nda_block_weights)", layer);
    if (nseq == 0)
        return NDA_OK;
    if (!x || !out || !aligned16(x) || !aligned16(out))
        return fail(c, NDA_ERR_ARG, "x / out null or not 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    const auto &w = c->blk[layer];
    const nda_config &g = c->cfg;
    // scratch parts, each a multiple of 4 floats (16-byte aligned): the two
    // prepared inputs in either form (the split one pads rows to 32 and adds
    // the row exponents), the projections at rows x their widths
    auto r4 = [](size_t n) { return (n + 3) & ~(size_t)3; };
    const size_t pxh = r4(nda_cq_split_bytes(w[0], nseq) / 4), pah = r4(nda_cq_split_bytes(w[4], nseq) / 4);
    const size_t nq = r4(w[0]->out), nk = r4(w[1]->out), nv = r4(w[2]->out), ng = r4(w[3]->out),
                 na = r4((size_t)g.n_heads * g.v_head_dim);
    if (int rc = ensure_buf(c, c->d_bscr, c->bscr_cap, pxh + (nq + nk + nv + ng + na) * nseq + pah))
        return rc;
    float *xh = c->d_bscr, *yq = xh + pxh, *yk = yq + nq * nseq, *yv = yk + nk * nseq,
          *yg = yv + nv * nseq, *att = yg + ng * nseq, *ah = att + na * nseq;
    // the parts are laid out [part][row] with row strides equal to the
    // tensors' own widths, as the kernels expect
    {
        ProfScope ps(c, NDA_K_PROJ, st);
        const nda_cq *ts[4] = {w[0], w[1], w[2], w[3]};
        float *ys[4] = {yq, yk, yv, yg};
        if (int rc = cq_project(ts, 4, nseq, x, xh, ys, st))
            return fail(c, rc, "q/k/v/gate projections");
    }
    int rc = c->taps ? nda_attention(c, layer, nseq, ids, yq, yk, yv, yg, att, stream)
                     : nda_step(c, layer, nseq, ids, yq, yk, yv, yg, att, stream);
    if (rc)
        return rc;
    ProfScope ps(c, NDA_K_PROJ, st);
    if (int rc2 = cq_project(&w[4], 1, nseq, att, ah, &out, st))
        return fail(c, rc2, "out_proj");
    return NDA_OK;
}

int nda_prefill_block(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens,
                      const float *x, float *out, void *stream)
{
    if (!c)
        return NDA_ERR_ARG;
    if (layer >= c->cfg.n_layers || c->blk.empty() || !c->blk[layer][0])
        return fail(c, NDA_ERR_STATE, "no projection weights for layer %u (nda_block_weights)", layer);
    if (nseq == 0)
        return NDA_OK;
    if (!n_tokens || !x || !out || !aligned16(x) || !aligned16(out))
        return fail(c, NDA_ERR_ARG, "n_tokens / x / out null, or x / out not 16-byte aligned");
    if (int rc = check_ids(c, nseq, ids))
        return rc;
    if (int rc = prefill_check(c, nseq, ids, n_tokens))
        return rc;
    if (c->taps)
        if (int rc = front_check(c, layer, nseq, ids, n_tokens))
            return rc;
    PrefillPlan pl;
    if (int rc = prefill_plan(c, nseq, ids, n_tokens, pl))
        return rc;
    const uint64_t rows = pl.rows;
    if (rows == 0)
        return NDA_OK;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = on_stream(c, st))
        return rc;
    const auto &w = c->blk[layer];
    const nda_config &g = c->cfg;
    // scratch parts as in nda_attention_block, plus the front's outputs
    auto r4 = [](size_t n) { return (n + 3) & ~(size_t)3; };
    const size_t pxh = r4(nda_cq_split_bytes(w[0], (uint32_t)rows) / 4),
                 pah = r4(nda_cq_split_bytes(w[4], (uint32_t)rows) / 4);
    const size_t nq = r4(w[0]->out), nk = r4(w[1]->out), nv = r4(w[2]->out), ng = r4(w[3]->out),
                 na = r4((size_t)g.n_heads * g.v_head_dim);
    const size_t nf = c->taps ? nq + nk + nv : 0;    // the front's outputs
    // Every buffer the pass needs (its scratch, the front's row lists and
    // history copies, the prefill's staging), then the pages: a call that
    // fails for want of memory or pages changes nothing, tap histories
    // included.
    if (int rc = ensure_buf(c, c->d_bscr, c->bscr_cap, pxh + (nq + nk + nv + ng + nf + na) * rows + pah))
        return rc;
    if (c->taps) {
        if (int rc = ensure_buf(c, c->d_front_rows, c->front_rows_cap, 3 * rows))
            return rc;
        if (int rc = hist_reserve(c, 0))
            return rc;
    }
    if (int rc = prefill_reserve(c, pl))
        return rc;
    {
        PageTxn txn(c->pt);
        for (uint32_t b = 0; b < nseq; b++) {
            const uint32_t qq = sid(ids, b);
            if (n_tokens[b])
                if (int rc = back_positions(c, qq, c->seqs[qq].pos, n_tokens[b]))
                    return rc;
        }
        txn.commit();
    }
    // [part][row], each part at its tensor's own row width
    float *xh = c->d_bscr, *yq = xh + pxh, *yk = yq + nq * rows, *yv = yk + nk * rows,
          *yg = yv + nv * rows, *fq = yg + ng * rows, *fk = fq + nq * rows, *fv = fk + nk * rows,
          *att = yg + (ng + nf) * rows, *ah = att + na * rows;
    const uint32_t nr = (uint32_t)rows;
    {
        ProfScope ps(c, NDA_K_PROJ, st);
        const nda_cq *ts[4] = {w[0], w[1], w[2], w[3]};
        float *ys[4] = {yq, yk, yv, yg};
        if (int rc = cq_project(ts, 4, nr, x, xh, ys, st))
            return fail(c, rc, "q/k/v/gate projections");
    }
    if (c->taps) {
        if (int rc = nda_front(c, layer, nseq, ids, n_tokens, yq, yk, yv, fq, fk, fv, stream))
            return rc;
        if (int rc = nda_prefill(c, layer, nseq, ids, n_tokens, fq, fk, fv, yg, att, stream))
            return rc;
    } else if (int rc = nda_prefill(c, layer, nseq, ids, n_tokens, yq, yk, yv, yg, att, stream)) {
        return rc;
    }
    ProfScope ps(c, NDA_K_PROJ, st);
    if (int rc = cq_project(&w[4], 1, nr, att, ah, &out, st))
        return fail(c, rc, "out_proj");
    return NDA_OK;
}

int nda_event_create(void **ev)
{
    if (!ev)
        return NDA_ERR_ARG;
    return hipEventCreate((hipEvent_t *)ev) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_event_destroy(void *ev) { return hipEventDestroy((hipEvent_t)ev) == hipSuccess ? NDA_OK : NDA_ERR_HIP; }

int nda_event_record(void *ev, void *stream)
{
    return hipEventRecord((hipEvent_t)ev, (hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_event_elapsed(void *start, void *stop, float *ms)
{
    if (!ms)
        return NDA_ERR_ARG;
    if (hipEventSynchronize((hipEvent_t)stop) != hipSuccess)
        return NDA_ERR_HIP;
    return hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_host_alloc(void **ptr, size_t bytes)
{
    if (!ptr)
        return NDA_ERR_ARG;
    hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault);
    return e == hipSuccess ? NDA_OK : (e == hipErrorOutOfMemory ? NDA_ERR_NOMEM : NDA_ERR_HIP);
}

int nda_host_free(void *ptr) { return hipHostFree(ptr) == hipSuccess ? NDA_OK : NDA_ERR_HIP; }

int nda_h2d_async(void *dst, const void *src, size_t bytes, void *stream)
{
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream) == hipSuccess
               ? NDA_OK
               : NDA_ERR_HIP;
}

int nda_d2h_async(void *dst, const void *src, size_t bytes, void *stream)
{
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream) == hipSuccess
               ? NDA_OK
               : NDA_ERR_HIP;
}

int nda_d2d(void *dst, const void *src, size_t bytes, void *stream)
{
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream) == hipSuccess
               ? NDA_OK
               : NDA_ERR_HIP;
}

int nda_memset(void *dst, int value, size_t bytes)
{
    return hipMemset(dst, value, bytes) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_fill_normal(void *dst, uint64_t n, int dtype, uint64_t seed, float scale, void *stream)
{
    if (!dst || (dtype != 0 && dtype != 1))
        return NDA_ERR_ARG;
    return launch_fill_normal(dst, n, dtype, seed, scale, (hipStream_t)stream) == hipSuccess ? NDA_OK
                                                                                             : NDA_ERR_HIP;
}

int nda_stream_create(void **stream)
{
    if (!stream)
        return NDA_ERR_ARG;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess)
        return NDA_ERR_HIP;
    *stream = s;
    return NDA_OK;
}

int nda_stream_destroy(void *stream)
{
    return hipStreamDestroy((hipStream_t)stream) == hipSuccess ? NDA_OK : NDA_ERR_HIP;
}

int nda_device_sync(void) { return hipDeviceSynchronize() == hipSuccess ? NDA_OK : NDA_ERR_HIP; }

int nda_device_info(char *name, size_t name_len, int *cu_count)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return NDA_ERR_NODEV;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess)
        return NDA_ERR_HIP;
    if (name && name_len) {
        snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    }
    if (cu_count)
        *cu_count = p.multiProcessorCount;
    return NDA_OK;
}

int nda_prof_enable(nda_ctx *c, int on)
{
    if (!c)
        return NDA_ERR_ARG;
    c->prof = on != 0;
    return NDA_OK;
}

int nda_prof_read(nda_ctx *c, double ms[NDA_K_COUNT], uint64_t launches[NDA_K_COUNT], int reset)
{
    if (!c)
        return NDA_ERR_ARG;
    for (auto &r : c->prof_pending) {
        float t = 0.0f;
        if (hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&t, r.a, r.b) == hipSuccess) {
            c->prof_ms[r.kind] += t;
            c->prof_n[r.kind]++;
        }
        c->ev_free.push_back(r.a);
        c->ev_free.push_back(r.b);
    }
    c->prof_pending.clear();
    for (int i = 0; i < NDA_K_COUNT; i++) {
        if (ms)
            ms[i] = c->prof_ms[i];
        if (launches)
            launches[i] = c->prof_n[i];
        if (reset) {
            c->prof_ms[i] = 0;
            c->prof_n[i] = 0;
        }
    }
    return NDA_OK;
}

} // extern "C"
