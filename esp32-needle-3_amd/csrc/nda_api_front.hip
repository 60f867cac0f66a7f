// nda_api_front.hip - the attention front of the C ABI (include/nda.h): tap
// histories, per-layer weights, the rotary table, nda_front and
// nda_attention (front + store + decode).
#include "nda_ctx.h"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

extern "C" {

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

} // extern "C"

namespace nda_host {

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

} // namespace nda_host

namespace {

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

extern "C" {

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

} // extern "C"
