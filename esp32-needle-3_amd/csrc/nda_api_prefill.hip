// nda_api_prefill.hip - causal prefill of the C ABI (include/nda.h): chunks
// of new tokens per sequence over the cached positions, planned into MFMA
// work items (or the per-row VALU path) and launched.
#include "nda_ctx.h"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

namespace nda_host {

int prefill_check(nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens)
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

int prefill_plan(nda_ctx *c, uint32_t nseq, const uint32_t *ids, const uint32_t *n_tokens, PrefillPlan &pl)
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
int prefill_reserve(nda_ctx *c, const PrefillPlan &pl)
{
    if (pl.rows == 0)
        return NDA_OK;
    if (pl.valu)
        return reserve_attend(c, (uint32_t)pl.rows, true, pl.max_total, pl.sum_total);
    if (int rc = ensure_rows(c, pl.rows))
        return rc;
    return ensure_pf(c, 8 * pl.n_items);
}

} // namespace nda_host

extern "C" {

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

} // extern "C"
