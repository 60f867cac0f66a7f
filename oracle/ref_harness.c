/* ref_harness.c - drives the reference engine's own attention code on
 * synthetic inputs, to pin the oracle restatement (nd_oracle.c).
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/ref.mk into oracle/_ref/ from the
 * reference sources where they lie (REF=/root/reference); no reference source
 * is copied into this repository. The engine's attention helpers are file-
 * static, so this translation unit includes engine/src/nd_model.c and reaches
 * them directly:
 *   kv_slot          engine/src/nd_model.c:1304-1309
 *   nd_model_set_sink / snapshot / rewind / prefix_*   :1314-1555
 *   kv_store_int8    :1822-1866
 *   attn_heads       :2105-2359
 * An nd_model is assembled by hand with only the KV geometry and buffers set
 * (no archive), and the store + dispatch steps of attention() (:2426-2483) are
 * replayed around those calls.
 */
#include "nd_model.c"

#include <stdio.h>

uint32_t ref_kv_slot(uint32_t window, uint32_t n_sink, uint32_t p)
{
    nd_model m;
    memset(&m, 0, sizeof m);
    m.window = window;
    m.n_sink = n_sink;
    return kv_slot(&m, p);
}

uint32_t ref_clamp_sink(uint32_t window, uint32_t n)
{
    nd_model m;
    memset(&m, 0, sizeof m);
    m.window = window;
    nd_model_set_sink(&m, n);
    return m.n_sink;
}

float ref_expf(float x) { return nd_expf(x); }

void ref_expf_pair(float x0, float x1, float *r0, float *r1) { nd_expf_pair(x0, x1, r0, r1); }

float ref_sigmoid(float x) { return sigmoidf_(x); }

void ref_sigmoid_pair(float x0, float x1, float *y0, float *y1) { sigmoidf_pair(x0, x1, y0, y1); }

void ref_kv_store_int8(int8_t *dst, const float *src, uint32_t n, float scale)
{
    kv_store_int8(dst, src, n, scale);
}

/* ---------------------------------------------------------------- session */

void *ref_session_new(uint32_t n_layers, uint32_t nh, uint32_t nkv, uint32_t qk_hd,
                      uint32_t v_hd, uint32_t window)
{
    nd_model *m = (nd_model *)calloc(1, sizeof *m);
    size_t slots = (size_t)n_layers * window;
    if (!m)
        return NULL;
    m->n_layers = n_layers;
    m->n_heads = nh;
    m->n_kv_heads = nkv;
    m->qk_head_dim = qk_hd;
    m->v_head_dim = v_hd;
    m->attn_dim = nh * v_hd;
    m->k_dim = nkv * qk_hd;
    m->v_dim = nkv * v_hd;
    m->window = window;
    m->k_cache = (int8_t *)calloc(slots * m->k_dim, 1);
    m->v_cache = (int8_t *)calloc(slots * m->v_dim, 1);
    m->k_scale = (float *)calloc(slots * nkv, sizeof(float));
    m->v_scale = (float *)calloc(slots * nkv, sizeof(float));
    m->q = (float *)calloc((size_t)nh * qk_hd, sizeof(float));
    m->gate = (float *)calloc((size_t)nh * v_hd, sizeof(float));
    m->attn = (float *)calloc((size_t)nh * v_hd, sizeof(float));
    m->kbuf = (float *)calloc(m->k_dim, sizeof(float));
    m->vbuf = (float *)calloc(m->v_dim, sizeof(float));
    return m;
}

void ref_session_free(void *vm)
{
    nd_model *m = (nd_model *)vm;
    if (!m)
        return;
    free(m->k_cache); free(m->v_cache); free(m->k_scale); free(m->v_scale);
    free(m->q); free(m->gate); free(m->attn); free(m->kbuf); free(m->vbuf);
    free(m->snap_eg_hist); free(m->snap_q_hist); free(m->snap_k_hist); free(m->snap_v_hist);
    free(m);
}

void ref_reset(void *vm) { nd_model_reset((nd_model *)vm); }
void ref_set_sink(void *vm, uint32_t n) { nd_model_set_sink((nd_model *)vm, n); }
int ref_snapshot(void *vm) { return nd_model_snapshot((nd_model *)vm); }
void ref_rewind(void *vm) { nd_model_rewind((nd_model *)vm); }
void *ref_prefix_save(void *vm) { return nd_model_prefix_save((nd_model *)vm); }
int ref_prefix_restore(void *vm, void *p) { return nd_model_prefix_restore((nd_model *)vm, (nd_prefix *)p); }
void ref_prefix_free(void *p) { nd_model_prefix_free((nd_prefix *)p); }
void ref_step_end(void *vm) { ((nd_model *)vm)->pos++; }
uint32_t ref_pos(void *vm) { return ((nd_model *)vm)->pos; }
uint32_t ref_n_sink(void *vm) { return ((nd_model *)vm)->n_sink; }
void ref_set_pos(void *vm, uint32_t p) { ((nd_model *)vm)->pos = p; }

void ref_cache(void *vm, int8_t **k, int8_t **v, float **ks, float **vs)
{
    nd_model *m = (nd_model *)vm;
    *k = m->k_cache; *v = m->v_cache; *ks = m->k_scale; *vs = m->v_scale;
}

/* Store k [nkv*qk_hd] / v [nkv*v_hd] at the current position's slot: the
 * per-kv-head absmax, the absmax/127 scale (1 for a zero row) and the
 * reference's kv_store_int8. */
void ref_kv_store(void *vm, uint32_t li, const float *k, const float *v)
{
    nd_model *m = (nd_model *)vm;
    size_t row = (size_t)li * m->window + kv_slot(m, m->pos);
    uint32_t g, i;
    for (g = 0; g < m->n_kv_heads; g++) {
        const float *kr = k + (size_t)g * m->qk_head_dim;
        const float *vr = v + (size_t)g * m->v_head_dim;
        float ak = 0.0f, av = 0.0f, sk, sv;
        for (i = 0; i < m->qk_head_dim; i++)
            ak = fabsf(kr[i]) > ak ? fabsf(kr[i]) : ak;
        for (i = 0; i < m->v_head_dim; i++)
            av = fabsf(vr[i]) > av ? fabsf(vr[i]) : av;
        sk = ak > 0.0f ? ak / 127.0f : 1.0f;
        sv = av > 0.0f ? av / 127.0f : 1.0f;
        m->k_scale[row * m->n_kv_heads + g] = sk;
        m->v_scale[row * m->n_kv_heads + g] = sv;
        kv_store_int8(m->k_cache + row * m->k_dim + (size_t)g * m->qk_head_dim, kr,
                      m->qk_head_dim, sk);
        kv_store_int8(m->v_cache + row * m->v_dim + (size_t)g * m->v_head_dim, vr,
                      m->v_head_dim, sv);
    }
}

/* Attend at the current position: the sink / recent run bounds of
 * attention() and one serial call of attn_heads over all heads (the host's
 * rows_serial splitter, engine/src/nd_quant.c:712-717). gate may be NULL
 * for "no output gate": the gate row is then +inf, whose sigmoid is exactly 1
 * (nd_expf saturates -inf to 0), so the emit leaves oh/denom unchanged. */
void ref_attend(void *vm, uint32_t li, const float *q, const float *gate, float *out)
{
    nd_model *m = (nd_model *)vm;
    attn_ctx c;
    uint32_t nh = m->n_heads, rcap = m->window - m->n_sink;

    memcpy(m->q, q, sizeof(float) * nh * m->qk_head_dim);
    if (gate)
        memcpy(m->gate, gate, sizeof(float) * nh * m->v_head_dim);
    else {
        uint32_t i;
        for (i = 0; i < nh * m->v_head_dim; i++)
            m->gate[i] = INFINITY;
    }
    c.m = m;
    c.li = li;
    c.nkv = m->n_kv_heads;
    c.rep = nh / m->n_kv_heads;
    c.nh = nh;
    c.qk_hd = m->qk_head_dim;
    c.v_hd = m->v_head_dim;
    c.scale = 1.0f / sqrtf((float)m->qk_head_dim);
    c.sinks = m->n_sink < m->pos + 1u ? m->n_sink : m->pos + 1u;
    if (m->pos + 1u <= m->n_sink) {
        c.rfirst = m->pos + 1u;
        c.rcount = 0;
    } else {
        c.rcount = m->pos + 1u - m->n_sink;
        if (c.rcount > rcap)
            c.rcount = rcap;
        c.rfirst = m->pos + 1u - c.rcount;
    }
    attn_heads(&c, 0, nh);
    memcpy(out, m->attn, sizeof(float) * nh * m->v_head_dim);
}

void ref_attention(void *vm, uint32_t li, const float *q, const float *k, const float *v,
                   const float *gate, float *out)
{
    ref_kv_store(vm, li, k, v);
    ref_attend(vm, li, q, gate, out);
}
