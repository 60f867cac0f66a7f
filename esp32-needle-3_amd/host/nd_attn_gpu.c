/* nd_attn_gpu.c - the engine-side C shim over libndattn (see nd_attn_gpu.h).
 *
 * One engine session = sequence 0 of a one-sequence context. Snapshot and
 * prefix caches map onto the library's shared prefix segments: a snapshot
 * builds a segment from the live KV, a saved prefix holds a reference to one,
 * and a restore attaches the session to it (a pointer switch on the device,
 * where the engine memcpy's every live slot back, nd_model.c:1543-1553).
 */
#include "nd_attn_gpu.h"

#include <stdlib.h>
#include <string.h>

struct nd_gpu_model {
    nda_ctx *ctx;
    uint32_t nh, nkv, qk_hd, v_hd, window;
    int has_snap;
    int32_t snap_prefix;      /* segment holding the snapshot's KV, -1 none */
    uint32_t snap_pos;
    /* Segments whose prefix handle was freed while the session still read
     * them; released once the session detaches. */
    int32_t orphan[64];
    uint32_t n_orphan;
    /* One token's q | k | v | gate, staged through page-locked host memory
     * in one copy each way; d_q.. point into d_in. */
    float *d_in, *d_q, *d_k, *d_v, *d_gate, *d_out;
    float *h_in, *h_out;
    size_t nq, nk, nv, ng;       /* floats */
    void *stream;
    /* the whole block (nd_gpu_block_weights): d_model-sized staging */
    uint32_t dm;
    float *d_x, *d_y, *h_x, *h_y;
};

struct nd_gpu_prefix {
    const nd_gpu_model *owner;
    int32_t segment;
    uint32_t pos;
};

nd_gpu_model *nd_gpu_open(uint32_t n_layers, uint32_t n_heads, uint32_t n_kv_heads,
                          uint32_t qk_head_dim, uint32_t v_head_dim, uint32_t window,
                          uint32_t kv_dtype, uint32_t max_prefixes)
{
    nda_config cfg;
    nd_gpu_model *m = (nd_gpu_model *)calloc(1, sizeof *m);
    if (!m)
        return NULL;
    memset(&cfg, 0, sizeof cfg);
    cfg.n_layers = n_layers;
    cfg.n_heads = n_heads;
    cfg.n_kv_heads = n_kv_heads;
    cfg.qk_head_dim = qk_head_dim;
    cfg.v_head_dim = v_head_dim;
    cfg.window = window;
    cfg.page_size = 16;
    cfg.kv_dtype = kv_dtype;
    cfg.max_seqs = 1;
    cfg.max_prefixes = max_prefixes ? max_prefixes + 1u : 8u;
    if (nda_create(&cfg, &m->ctx) != NDA_OK) {
        free(m);
        return NULL;
    }
    m->nh = n_heads;
    m->nkv = n_kv_heads;
    m->qk_hd = qk_head_dim;
    m->v_hd = v_head_dim;
    m->window = window;
    m->snap_prefix = -1;
    /* each part rounded to 4 floats keeps every part 16-byte aligned */
    m->nq = ((size_t)n_heads * qk_head_dim + 3) & ~(size_t)3;
    m->nk = ((size_t)n_kv_heads * qk_head_dim + 3) & ~(size_t)3;
    m->nv = ((size_t)n_kv_heads * v_head_dim + 3) & ~(size_t)3;
    m->ng = ((size_t)n_heads * v_head_dim + 3) & ~(size_t)3;
    if (nda_stream_create(&m->stream) ||
        nda_dev_alloc((void **)&m->d_in, sizeof(float) * (m->nq + m->nk + m->nv + m->ng)) ||
        nda_dev_alloc((void **)&m->d_out, sizeof(float) * m->ng) ||
        nda_host_alloc((void **)&m->h_in, sizeof(float) * (m->nq + m->nk + m->nv + m->ng)) ||
        nda_host_alloc((void **)&m->h_out, sizeof(float) * m->ng)) {
        nd_gpu_close(m);
        return NULL;
    }
    m->d_q = m->d_in;
    m->d_k = m->d_q + m->nq;
    m->d_v = m->d_k + m->nk;
    m->d_gate = m->d_v + m->nv;
    return m;
}

void nd_gpu_close(nd_gpu_model *m)
{
    if (!m)
        return;
    if (m->d_in)
        nda_dev_free(m->d_in);
    if (m->d_out)
        nda_dev_free(m->d_out);
    if (m->h_in)
        nda_host_free(m->h_in);
    if (m->h_out)
        nda_host_free(m->h_out);
    if (m->d_x)
        nda_dev_free(m->d_x);
    if (m->d_y)
        nda_dev_free(m->d_y);
    if (m->h_x)
        nda_host_free(m->h_x);
    if (m->h_y)
        nda_host_free(m->h_y);
    nda_destroy(m->ctx);
    if (m->stream)
        nda_stream_destroy(m->stream);
    free(m);
}

nda_ctx *nd_gpu_ctx(nd_gpu_model *m) { return m->ctx; }

uint32_t nd_gpu_pos(const nd_gpu_model *m)
{
    uint32_t pos = 0;
    nda_seq_state(m->ctx, 0, &pos, NULL, NULL);
    return pos;
}

uint32_t nd_gpu_n_sink(const nd_gpu_model *m)
{
    uint32_t n = 0;
    nda_seq_state(m->ctx, 0, NULL, &n, NULL);
    return n;
}

/* Free orphaned segments the session no longer reads. */
static void sweep_orphans(nd_gpu_model *m)
{
    uint32_t i, kept = 0;
    for (i = 0; i < m->n_orphan; i++)
        if (nda_prefix_free(m->ctx, m->orphan[i]) != NDA_OK)
            m->orphan[kept++] = m->orphan[i];
    m->n_orphan = kept;
}

static void orphan(nd_gpu_model *m, int32_t seg)
{
    if (seg < 0)
        return;
    if (nda_prefix_free(m->ctx, seg) == NDA_OK)
        return;
    if (m->n_orphan < sizeof m->orphan / sizeof m->orphan[0])
        m->orphan[m->n_orphan++] = seg;
}

void nd_gpu_reset(nd_gpu_model *m)
{
    nda_seq_reset(m->ctx, 0);
    orphan(m, m->snap_prefix);
    m->snap_prefix = -1;
    m->has_snap = 0;
    sweep_orphans(m);
}

void nd_gpu_set_sink(nd_gpu_model *m, uint32_t n)
{
    nda_seq_set_sink(m->ctx, 0, n);
}

/* The snapshot pins pos as sinks and keeps the KV up to pos in a segment;
 * the session then continues attached to that segment. */
int nd_gpu_snapshot(nd_gpu_model *m)
{
    int32_t id = -1;
    int32_t old = m->snap_prefix;
    if (nda_prefix_build(m->ctx, 0, &id, m->stream) != NDA_OK)
        return -1;
    if (nda_seq_attach(m->ctx, 0, id, m->stream) != NDA_OK) {
        nda_prefix_free(m->ctx, id);
        return -1;
    }
    orphan(m, old);
    sweep_orphans(m);
    m->snap_prefix = id;
    m->snap_pos = nd_gpu_pos(m);
    m->has_snap = 1;
    return 0;
}

void nd_gpu_rewind(nd_gpu_model *m)
{
    if (!m->has_snap) {
        nd_gpu_reset(m);
        return;
    }
    nda_seq_rewind(m->ctx, 0);
}

nd_gpu_prefix *nd_gpu_prefix_save(nd_gpu_model *m)
{
    nd_gpu_prefix *p;
    if (!m->has_snap || nd_gpu_pos(m) != m->snap_pos)
        return NULL;
    p = (nd_gpu_prefix *)malloc(sizeof *p);
    if (!p)
        return NULL;
    p->owner = m;
    p->segment = m->snap_prefix;
    p->pos = m->snap_pos;
    m->snap_prefix = -1;      /* the saved prefix now owns the segment */
    return p;
}

int nd_gpu_prefix_restore(nd_gpu_model *m, const nd_gpu_prefix *p)
{
    int32_t old;
    if (!p || p->owner != m)
        return -1;
    old = m->snap_prefix;
    if (nda_seq_attach(m->ctx, 0, p->segment, m->stream) != NDA_OK)
        return -1;
    if (old != p->segment)
        orphan(m, old);
    m->snap_prefix = -1;
    sweep_orphans(m);
    m->has_snap = 1;
    m->snap_pos = p->pos;
    return 0;
}

void nd_gpu_prefix_free(nd_gpu_prefix *p)
{
    if (!p)
        return;
    /* A segment the session still reads is released when it detaches. */
    orphan((nd_gpu_model *)p->owner, p->segment);
    free(p);
}

/* One layer call on host arrays: stage q | k | v | gate into page-locked
 * memory, one copy in, the launches, one copy out, one wait. raw selects the
 * front (raw projections) or the post-front entry. */
static int attend_host(nd_gpu_model *m, int raw, uint32_t li, const float *q, const float *k,
                       const float *v, const float *gate, float *out)
{
    size_t n = m->nq + m->nk + m->nv + (gate ? m->ng : 0);
    size_t vh = (size_t)m->nh * m->v_hd;
    int rc;
    memcpy(m->h_in, q, sizeof(float) * m->nh * m->qk_hd);
    memcpy(m->h_in + m->nq, k, sizeof(float) * m->nkv * m->qk_hd);
    memcpy(m->h_in + m->nq + m->nk, v, sizeof(float) * m->nkv * m->v_hd);
    if (gate)
        memcpy(m->h_in + m->nq + m->nk + m->nv, gate, sizeof(float) * vh);
    rc = nda_h2d_async(m->d_in, m->h_in, sizeof(float) * n, m->stream);
    if (rc)
        return rc;
    if (raw)
        rc = nda_attention(m->ctx, li, 1, NULL, m->d_q, m->d_k, m->d_v, gate ? m->d_gate : NULL,
                           m->d_out, m->stream);
    else
        rc = nda_step(m->ctx, li, 1, NULL, m->d_q, m->d_k, m->d_v, gate ? m->d_gate : NULL,
                      m->d_out, m->stream);
    if (rc)
        return rc;
    rc = nda_d2h_async(m->h_out, m->d_out, sizeof(float) * vh, m->stream);
    if (rc)
        return rc;
    rc = nda_sync(m->ctx, m->stream);
    if (rc)
        return rc;
    memcpy(out, m->h_out, sizeof(float) * vh);
    return 0;
}

int nd_gpu_attention(nd_gpu_model *m, uint32_t li, const float *q, const float *k,
                     const float *v, const float *gate, float *out)
{
    return attend_host(m, 0, li, q, k, v, gate, out);
}

int nd_gpu_front_init(nd_gpu_model *m, uint32_t taps, float rope_theta, uint32_t max_pos)
{
    nda_front_config fc;
    fc.taps = taps;
    fc.rope_theta = rope_theta;
    fc.max_pos = max_pos;
    return nda_front_init(m->ctx, &fc);
}

int nd_gpu_front_weights(nd_gpu_model *m, uint32_t li, const float *tap_q, const float *tap_k,
                         const float *tap_v, const float *norm_q, const float *norm_k)
{
    return nda_front_weights(m->ctx, li, tap_q, tap_k, tap_v, norm_q, norm_k);
}

int nd_gpu_attention_raw(nd_gpu_model *m, uint32_t li, const float *q, const float *k,
                         const float *v, const float *gate, float *out)
{
    return attend_host(m, 1, li, q, k, v, gate, out);
}

int nd_gpu_block_weights(nd_gpu_model *m, uint32_t li, const nda_cq *q, const nda_cq *k, const nda_cq *v,
                         const nda_cq *gate, const nda_cq *out_proj)
{
    int rc = nda_block_weights(m->ctx, li, q, k, v, gate, out_proj);
    uint32_t dm = 0;
    if (rc)
        return rc;
    dm = nda_cq_in_pad(q);     /* >= d_model; the staging holds either */
    if (m->dm >= dm)
        return 0;
    if (m->d_x) { nda_dev_free(m->d_x); m->d_x = NULL; }
    if (m->d_y) { nda_dev_free(m->d_y); m->d_y = NULL; }
    if (m->h_x) { nda_host_free(m->h_x); m->h_x = NULL; }
    if (m->h_y) { nda_host_free(m->h_y); m->h_y = NULL; }
    m->dm = 0;
    if (nda_dev_alloc((void **)&m->d_x, sizeof(float) * dm) ||
        nda_dev_alloc((void **)&m->d_y, sizeof(float) * dm) ||
        nda_host_alloc((void **)&m->h_x, sizeof(float) * dm) ||
        nda_host_alloc((void **)&m->h_y, sizeof(float) * dm))
        return NDA_ERR_NOMEM;
    m->dm = dm;
    return 0;
}

int nd_gpu_attention_block(nd_gpu_model *m, uint32_t li, const float *xin, uint32_t d_model, float *out)
{
    int rc;
    if (!m->dm || d_model > m->dm)
        return NDA_ERR_STATE;
    memcpy(m->h_x, xin, sizeof(float) * d_model);
    rc = nda_h2d_async(m->d_x, m->h_x, sizeof(float) * d_model, m->stream);
    if (rc)
        return rc;
    rc = nda_attention_block(m->ctx, li, 1, NULL, m->d_x, m->d_y, m->stream);
    if (rc)
        return rc;
    rc = nda_d2h_async(m->h_y, m->d_y, sizeof(float) * d_model, m->stream);
    if (rc)
        return rc;
    rc = nda_sync(m->ctx, m->stream);
    if (rc)
        return rc;
    memcpy(out, m->h_y, sizeof(float) * d_model);
    return 0;
}

void nd_gpu_step_end(nd_gpu_model *m)
{
    nda_advance(m->ctx, 1, NULL, 1, m->stream);
}
