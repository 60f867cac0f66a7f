// nda_api_decode.hip - the decode calls of the C ABI (include/nda.h): KV
// append, single-token attention (split-KV with its merge, the shared-prefix
// pass, GQA groups on MFMA), the fused store + attention step and the
// allocation-free decode, and the launch of the decode kernels.
#include "nda_ctx.h"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

namespace nda_host {

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
int run_attend(nda_ctx *c, AttnArgs &a, hipStream_t st, float *part, bool prof, bool ordered)
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

} // namespace nda_host

extern "C" {

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

} // extern "C"

namespace nda_host {

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
// tile. A fused append stores in the own pass (the work-group whose chunk
// holds the new slot, as in a single pass); the prefix pass reads no own
// slot. Rows longer than
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

// whether a batch's sequences qualify (see above); max_total (may be null):
// the longest visible run
static bool prefix_split_batch(const nda_ctx *c, uint32_t nseq, const uint32_t *ids, int32_t *pfx_out,
                               uint32_t *nsh_out, uint32_t *max_total)
{
    if (nseq == 0 || mfma_decode_geo(c) || !prefill_mfma_supported(c->geo) ||
        (c->cfg.flags & (NDA_FLAG_PREFILL_VALU | NDA_FLAG_DECODE_VALU)))
        return false;
    if ((uint64_t)nseq * c->cfg.n_kv_heads < 4ull * (uint64_t)c->cus)
        return false;
    int32_t pfx = -1;
    uint32_t nsh = 0, mt = 0;
    for (uint32_t b = 0; b < nseq; b++) {
        const SeqHost &s = c->seqs[sid(ids, b)];
        if (s.prefix < 0)
            return false;
        const Vis v = visible(s, s.pos, c->cfg.window);
        mt = std::max(mt, v.n_sh + v.n_own);
        if (b == 0) {
            pfx = s.prefix;
            nsh = v.n_sh;
        } else if (s.prefix != pfx || v.n_sh != nsh) {
            return false;
        }
    }
    *pfx_out = pfx;
    *nsh_out = nsh;
    if (max_total)
        *max_total = mt;
    return nsh >= 32;
}

// whether the pass is taken: a qualifying batch whose rows run past the
// prefix by at most PREFIX_PASS_MAX_CHUNKS - 1 prefix lengths
static bool prefix_split_on(uint32_t nsh, uint32_t max_total)
{
    return max_total > nsh && (max_total + nsh - 1) / nsh <= PREFIX_PASS_MAX_CHUNKS;
}

static void prefix_split_plan(nda_ctx *c, uint32_t nseq, const uint32_t *ids, uint32_t max_total,
                              PrefixSplit &ps)
{
    ps = PrefixSplit();
    int32_t pfx;
    uint32_t nsh;
    if (!prefix_split_batch(c, nseq, ids, &pfx, &nsh, nullptr) || !prefix_split_on(nsh, max_total))
        return;
    const uint32_t chunks = (max_total + nsh - 1) / nsh;
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
static int decode_reserve(nda_ctx *c, uint32_t nseq, const uint32_t *ids, uint32_t max_total,
                          uint64_t sum_total, PrefixSplit &psp)
{
    if (int rc = reserve_attend(c, nseq, ids != nullptr, max_total, sum_total))
        return rc;
    prefix_split_plan(c, nseq, ids, max_total, psp);
    if (psp.on) {
        if (int rc = ensure_part(c, (size_t)nseq * c->cfg.n_heads * psp.max_chunks * (c->cfg.v_head_dim + 2)))
            return rc;
        if (int rc = ensure_pf(c, 8 * (size_t)psp.n_items))
            return rc;
    }
    return NDA_OK;
}

int decode_impl(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
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
    if (int rc = decode_reserve(c, nseq, ids, max_total, sum_total, psp))
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

} // namespace nda_host

extern "C" {


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
// 4 work items per CU. Batches on one shared prefix that its decode pass
// serves fuse the store into the own-positions pass: about the same GPU
// time as a separate append (1024 sequences on a 213-token prefix: 53.6-56.2
// against 54.4 us per layer step), one launch fewer to enqueue (whole steps
// 1.65-1.70 M against 1.23-1.45 M tokens/s, host-bound).
int nda_step(nda_ctx *c, uint32_t layer, uint32_t nseq, const uint32_t *ids, const float *q,
             const float *k, const float *v, const float *gate, float *out, void *stream)
{
    if (c && nseq && (!k || !v))
        return fail(c, NDA_ERR_ARG, "null k/v");
    const uint64_t units = c ? (uint64_t)nseq * c->cfg.n_kv_heads : 0;
    int32_t pfx;
    uint32_t nsh, mt;
    if (c && layer < c->cfg.n_layers && check_ids(c, nseq, ids) == NDA_OK &&
        prefix_split_batch(c, nseq, ids, &pfx, &nsh, &mt) && prefix_split_on(nsh, mt))
        return decode_impl(c, layer, nseq, ids, q, k, v, gate, out, stream);
    if (c && (units >= 16ull * (uint64_t)c->cus || (mfma_decode_geo(c) && units >= 4ull * (uint64_t)c->cus))) {
        // The decode's buffers first: once the append has stored this
        // position, a decode that fails for want of memory would leave the
        // step half done.
        if (layer < c->cfg.n_layers && check_ids(c, nseq, ids) == NDA_OK) {
            uint32_t max_total;
            uint64_t sum_total;
            decode_totals(c, nseq, ids, &max_total, &sum_total);
            PrefixSplit psp;
            if (int rc = decode_reserve(c, nseq, ids, max_total, sum_total, psp))
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

} // extern "C"
