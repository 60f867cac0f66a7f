// nda_api_ctx.hip - libndattn's context: creation and teardown, device
// buffers and the pinned upload ring, per-sequence state and shared prefix
// segments, KV inspection, and the memory / stream / device calls of the C
// ABI (include/nda.h).
#include "nda_ctx.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_set>

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

} // namespace

namespace nda_host {

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

// row_seq | row_t staging for `rows` rows
int ensure_rows(nda_ctx *c, size_t rows)
{
    return grow_buf(c, c->d_rows, c->rows_cap, rows * 2, std::max<size_t>(rows * 2, 8192));
}

int ensure_part(nda_ctx *c, size_t floats) { return grow_buf(c, c->d_part, c->part_cap, floats, floats); }

int ensure_pf(nda_ctx *c, size_t n) { return grow_buf(c, c->d_pf, c->pf_cap, n, std::max<size_t>(n * 2, 16384)); }

int ensure_stage(nda_ctx *c, size_t bytes) { return grow_buf(c, c->d_stage, c->stage_cap, bytes, bytes); }

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

} // namespace nda_host

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
