/* ref_engine_gpu.c - the engine-side binding of libndhost, compiled against
 * the reference engine's own headers and sources and linked against
 * esp32-needle-3_amd/libndhost.so: the drop-in checked at build level and
 * run against the engine's CPU attention.
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/ref.mk into oracle/_ref/ from the
 * reference sources where they lie; no reference source is copied into this
 * repository. It includes ref_harness.c (which includes
 * engine/src/nd_model.c) for the hand-assembled nd_model and the replayed
 * store + attn_heads dispatch of attention() (nd_model.c:2426-2483).
 *
 * The binding is what an engine maintainer adds:
 *   - a GPU session beside the nd_model (a field of nd_model in the engine;
 *     here a wrapper, since the header is not edited);
 *   - in attention(), one nd_gpu_attention call on the engine's own buffers
 *     m->q, m->kbuf, m->vbuf, m->gate into m->attn, in place of the store
 *     and the attn_heads dispatch;
 *   - in nd_model_reset / _set_sink / _snapshot / _rewind / _prefix_save /
 *     _prefix_restore / _prefix_free and the position step of
 *     nd_model_step_hidden (m->pos++, nd_model.c:3094), the matching nd_gpu_*
 *     call (engine/include/nd_model.h:193-222);
 *   - for the whole attention() on the GPU: the front's tap count, theta and
 *     staged weights (fp16_slot[li][4..8]) handed over once, each layer's
 *     five CQ tensors registered from the archive's own blobs and codebook
 *     (nd_cact_data, nd_cact_codebook), and attention(m, li, xin, out)
 *     becoming one nd_gpu_attention_block call.
 * Each eng_* call below runs the engine's own body and the binding's call
 * side by side, so one token stream drives the CPU attention and the GPU
 * drop-in through the same nd_model.
 */
#include "ref_harness.c"

#include "nd_attn_gpu.h"

typedef struct {
    nd_model *m;
    nd_gpu_model *gpu;
    uint32_t d_model;
    nda_cq **cq;        /* [layer * 5 + tensor], registered with the session */
} eng;

typedef struct {
    nd_prefix *cpu;
    nd_gpu_prefix *gpu;
} eng_prefix;

void *eng_open(uint32_t n_layers, uint32_t nh, uint32_t nkv, uint32_t qk_hd, uint32_t v_hd, uint32_t window)
{
    eng *e = (eng *)calloc(1, sizeof *e);
    if (!e)
        return NULL;
    e->m = (nd_model *)ref_session_new(n_layers, nh, nkv, qk_hd, v_hd, window);
    /* nd_model_open: the session, int8 K/V as the engine stores them, 8
     * prefix segments */
    e->gpu = nd_gpu_open(n_layers, nh, nkv, qk_hd, v_hd, window, NDA_KV_INT8, 8);
    if (!e->m || !e->gpu) {
        if (e->gpu)
            nd_gpu_close(e->gpu);
        ref_session_free(e->m);
        free(e);
        return NULL;
    }
    return e;
}

void eng_close(void *ve)
{
    eng *e = (eng *)ve;
    uint32_t i;
    if (!e)
        return;
    nd_gpu_close(e->gpu);
    if (e->cq)      /* the tensors outlive the session that uses them */
        for (i = 0; i < e->m->n_layers * 5; i++)
            if (e->cq[i])
                nda_cq_destroy(e->cq[i]);
    free(e->cq);
    ref_session_free(e->m);
    free(e);
}

/* attention() of layer li at the model's position with q/k/v/gate as the
 * projections (and front) leave them in the engine's buffers. cpu_out: the
 * engine's store + attn_heads dispatch; gpu_out: the binding's single call.
 * Returns the call's status (0 or a negative NDA_ERR_* code). gate may be
 * NULL (no output gate). */
int eng_attention(void *ve, uint32_t li, const float *q, const float *k, const float *v, const float *gate,
                  float *cpu_out, float *gpu_out)
{
    eng *e = (eng *)ve;
    nd_model *m = e->m;
    const uint32_t nh = m->n_heads;
    int rc;
    ref_attention(m, li, q, k, v, gate, cpu_out);
    /* the buffers attention() holds at its store (nd_model.c:2426) */
    memcpy(m->q, q, sizeof(float) * nh * m->qk_head_dim);
    memcpy(m->kbuf, k, sizeof(float) * m->k_dim);
    memcpy(m->vbuf, v, sizeof(float) * m->v_dim);
    if (gate)
        memcpy(m->gate, gate, sizeof(float) * nh * m->v_head_dim);
    /* the binding */
    rc = nd_gpu_attention(e->gpu, li, m->q, m->kbuf, m->vbuf, gate ? m->gate : NULL, m->attn);
    memcpy(gpu_out, m->attn, sizeof(float) * nh * m->v_head_dim);
    return rc;
}

void eng_step_end(void *ve)
{
    eng *e = (eng *)ve;
    e->m->pos++;
    nd_gpu_step_end(e->gpu);
}

void eng_reset(void *ve)
{
    eng *e = (eng *)ve;
    nd_model_reset(e->m);
    nd_gpu_reset(e->gpu);
}

void eng_set_sink(void *ve, uint32_t n)
{
    eng *e = (eng *)ve;
    nd_model_set_sink(e->m, n);
    nd_gpu_set_sink(e->gpu, n);
}

/* both results: the engine's in *cpu, the session's in *gpu */
void eng_snapshot(void *ve, int *cpu, int *gpu)
{
    eng *e = (eng *)ve;
    *cpu = nd_model_snapshot(e->m);
    *gpu = nd_gpu_snapshot(e->gpu);
}

void eng_rewind(void *ve)
{
    eng *e = (eng *)ve;
    nd_model_rewind(e->m);
    nd_gpu_rewind(e->gpu);
}

void *eng_prefix_save(void *ve)
{
    eng *e = (eng *)ve;
    eng_prefix *p = (eng_prefix *)calloc(1, sizeof *p);
    if (!p)
        return NULL;
    p->cpu = nd_model_prefix_save(e->m);
    p->gpu = nd_gpu_prefix_save(e->gpu);
    if (!p->cpu || !p->gpu) {
        nd_model_prefix_free(p->cpu);
        nd_gpu_prefix_free(p->gpu);
        free(p);
        return NULL;
    }
    return p;
}

void eng_prefix_restore(void *ve, void *vp, int *cpu, int *gpu)
{
    eng *e = (eng *)ve;
    eng_prefix *p = (eng_prefix *)vp;
    *cpu = nd_model_prefix_restore(e->m, p->cpu);
    *gpu = nd_gpu_prefix_restore(e->gpu, p->gpu);
}

void eng_prefix_free(void *vp)
{
    eng_prefix *p = (eng_prefix *)vp;
    if (!p)
        return;
    nd_model_prefix_free(p->cpu);
    nd_gpu_prefix_free(p->gpu);
    free(p);
}

/* positions and sink counts of both sides */
void eng_state(void *ve, uint32_t *pos_cpu, uint32_t *sink_cpu, uint32_t *pos_gpu, uint32_t *sink_gpu)
{
    eng *e = (eng *)ve;
    *pos_cpu = e->m->pos;
    *sink_cpu = e->m->n_sink;
    *pos_gpu = nd_gpu_pos(e->gpu);
    *sink_gpu = nd_gpu_n_sink(e->gpu);
}

/* ------------------------------------------------- the whole attention() */

/* The attention front on both sides: the tap histories and rotary
 * frequencies nd_model_open sets up, and the session's nd_gpu_front_init. */
int eng_front(void *ve, uint32_t taps, float theta)
{
    eng *e = (eng *)ve;
    if (ref_session_front(e->m, taps, theta))
        return -1;
    return nd_gpu_front_init(e->gpu, taps, theta, 0);
}

/* The engine's nd_layer CQ tensors over one nd_cact buffer (blobs[layer * 5
 * + t], t = q, k, v, gate, out_proj; the archive's 28-float codebook) and
 * its staged front weights front[layer * 5 + i] (tap_q, tap_k, tap_v, norm_q,
 * norm_k in fp16_slot[li][4..8]); then, as the binding registers them, each
 * layer's front weights and one nda_cq per tensor made from the archive's
 * own blob and codebook slice. */
int eng_block_setup(void *ve, uint32_t d_model, uint32_t group, const void *const *blobs, const float *codebook,
                    const float *const *front)
{
    eng *e = (eng *)ve;
    nd_model *m = e->m;
    uint32_t li, i;
    if (ref_block_setup(m, d_model, group, blobs, codebook))
        return -1;
    e->d_model = d_model;
    e->cq = (nda_cq **)calloc((size_t)m->n_layers * 5, sizeof(nda_cq *));
    if (!e->cq)
        return -1;
    for (li = 0; li < m->n_layers; li++) {
        const nd_layer *L = &m->layer[li];
        const nd_tensor *src[5] = { &L->q_proj, &L->k_proj, &L->v_proj, &L->gate_proj, &L->out_proj };
        nda_cq **t = e->cq + (size_t)li * 5;
        int rc;
        for (i = 0; i < 5; i++)
            m->fp16_slot[li][4 + i] = (float *)front[li * 5 + i];
        rc = nd_gpu_front_weights(e->gpu, li, m->fp16_slot[li][4], m->fp16_slot[li][5], m->fp16_slot[li][6],
                                  m->fp16_slot[li][7], m->fp16_slot[li][8]);
        if (rc)
            return rc;
        for (i = 0; i < 5; i++) {
            rc = nda_cq_create(src[i]->shape[0], src[i]->shape[1], src[i]->group, src[i]->bits,
                               nd_cact_data(&m->c, src[i]), nd_cact_codebook(&m->c, src[i]->bits), &t[i]);
            if (rc)
                return rc;
        }
        rc = nd_gpu_block_weights(e->gpu, li, t[0], t[1], t[2], t[3], t[4]);
        if (rc)
            return rc;
    }
    return 0;
}

/* attention(m, li, xin, out) at the model's position: cpu_out from the
 * engine's own function (with the rotary table of nd_model_step_hidden),
 * gpu_out from the binding's single call. Returns the call's status. */
int eng_attention_block(void *ve, uint32_t li, const float *xin, float *cpu_out, float *gpu_out)
{
    eng *e = (eng *)ve;
    nd_model *m = e->m;
    ref_attention_block(m, li, m->fp16_slot[li][4], m->fp16_slot[li][5], m->fp16_slot[li][6], m->fp16_slot[li][7],
                        m->fp16_slot[li][8], xin, cpu_out);
    return nd_gpu_attention_block(e->gpu, li, xin, e->d_model, gpu_out);
}
