// nda_api_cq.hip - CQ projections and the attention block calls of the C ABI
// (include/nda.h): codebook-quantised tensors on the device, their matvecs
// in the three forms, and nda_attention_block / nda_prefill_block.
#include "nda_ctx.h"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

extern "C" {

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

} // extern "C"
