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
 *   tap_projection / tap_rows, zcrms_heads   :2361-2379, :1748-1802, :324-360
 * and the CQ kernels of engine/src/nd_quant.c (nd_fwht, nd_cq_prepare,
 * nd_cq_gemv_prepared, nd_cq_lut_build, nd_cq_gemv_lut2), driven with
 * hand-built nd_tensor / nd_cact records.
 * An nd_model is assembled by hand with only the KV geometry and buffers set
 * (no archive), and the store + dispatch steps of attention() (:2426-2483) are
 * replayed around those calls.
 */
#include "nd_model.c"

#include <pthread.h>
#include <stdio.h>
#include <time.h>

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
    free(m->q_hist); free(m->k_hist); free(m->v_hist);
    free(m->rope_inv); free(m->rope_cos); free(m->rope_sin);
    free(m->xh); free(m->lut); free(m->layer); free((void *)m->c.base);
    free(m);
}

/* ------------------------------------------------------ attention front */

/* Give the hand-built model the attention-front state nd_model_open sets up:
 * qkv_conv_taps, the tap histories [layer][tap][dim] (nd_model.c:1178-1180)
 * and the rotary inverse frequencies (:1233-1236, restated here because
 * nd_model_open needs an archive). */
int ref_session_front(void *vm, uint32_t taps, float theta)
{
    nd_model *m = (nd_model *)vm;
    uint32_t i, half = m->qk_head_dim / 2;
    m->c.h.qkv_conv_taps = taps;
    m->c.h.rope_theta = theta;
    m->q_hist = (float *)calloc((size_t)m->n_layers * taps * m->n_heads * m->qk_head_dim, sizeof(float));
    m->k_hist = (float *)calloc((size_t)m->n_layers * taps * m->k_dim, sizeof(float));
    m->v_hist = (float *)calloc((size_t)m->n_layers * taps * m->v_dim, sizeof(float));
    m->rope_inv = (float *)calloc(half + 1, sizeof(float));
    m->rope_cos = (float *)calloc(half + 1, sizeof(float));
    m->rope_sin = (float *)calloc(half + 1, sizeof(float));
    if (!m->q_hist || !m->k_hist || !m->v_hist || !m->rope_inv || !m->rope_cos || !m->rope_sin)
        return -1;
    for (i = 0; i < half; i++)
        m->rope_inv[i] = 1.0f / powf(theta, (float)(2 * i) / (float)m->qk_head_dim);
    return 0;
}

/* The front of attention() for layer li at the model's pos (nd_model.c:
 * 2413-2424) on raw q/k/v, in place: the per-position rotary table of
 * nd_model_step_hidden (:2949-2954, restated), then the reference's own
 * tap_projection x3 and zcrms_heads x2 with the given per-layer weights in
 * the engine's fp16_slot[li][4..8]. */
void ref_front(void *vm, uint32_t li, const float *tap_q, const float *tap_k, const float *tap_v,
               const float *norm_q, const float *norm_k, float *q, float *k, float *v)
{
    nd_model *m = (nd_model *)vm;
    uint32_t i, nh = m->n_heads, qk = m->qk_head_dim;
    for (i = 0; i < qk / 2; i++) {
        float angle = (float)m->pos * m->rope_inv[i];
        m->rope_cos[i] = cosf(angle);
        m->rope_sin[i] = sinf(angle);
    }
    m->fp16_slot[li][4] = (float *)tap_q;
    m->fp16_slot[li][5] = (float *)tap_k;
    m->fp16_slot[li][6] = (float *)tap_v;
    m->fp16_slot[li][7] = (float *)norm_q;
    m->fp16_slot[li][8] = (float *)norm_k;
    memcpy(m->q, q, sizeof(float) * nh * qk);
    memcpy(m->kbuf, k, sizeof(float) * m->k_dim);
    memcpy(m->vbuf, v, sizeof(float) * m->v_dim);
    tap_projection(m, 4, m->q, m->q_hist, li, nh * qk);
    tap_projection(m, 5, m->kbuf, m->k_hist, li, m->k_dim);
    tap_projection(m, 6, m->vbuf, m->v_hist, li, m->v_dim);
    zcrms_heads(m, m->fp16_slot[li][7], m->rope_cos, m->rope_sin, m->q, nh, qk);
    zcrms_heads(m, m->fp16_slot[li][8], m->rope_cos, m->rope_sin, m->kbuf, m->n_kv_heads, qk);
    memcpy(q, m->q, sizeof(float) * nh * qk);
    memcpy(k, m->kbuf, sizeof(float) * m->k_dim);
    memcpy(v, m->vbuf, sizeof(float) * m->v_dim);
}

/* The reference's own tap histories (live, or the snapshot's). */
void ref_hist(void *vm, int snap, float **q, float **k, float **v)
{
    nd_model *m = (nd_model *)vm;
    *q = snap ? m->snap_q_hist : m->q_hist;
    *k = snap ? m->snap_k_hist : m->k_hist;
    *v = snap ? m->snap_v_hist : m->v_hist;
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

/* ------------------------------------------------------- CQ projections */

void ref_fwht(float *x, uint32_t n) { nd_fwht(x, n); }

static void cq_tensor(nd_tensor *t, uint32_t out, uint32_t in, uint32_t group, uint32_t bits)
{
    memset(t, 0, sizeof *t);
    t->ndim = 2;
    t->shape[0] = out;
    t->shape[1] = in;
    t->group = group;
    t->bits = bits;
}

void ref_cq_prepare(uint32_t in, uint32_t group, const float *x, float *xh)
{
    nd_tensor t;
    cq_tensor(&t, 1, in, group, 2);
    nd_cq_prepare(&t, x, xh);
}

/* codebook: the archive's 28 floats cb2 | cb3 | cb4 (nd_cact_codebook). */
void ref_cq_gemv(uint32_t out, uint32_t in, uint32_t group, uint32_t bits, const void *blob,
                 const float *codebook, const float *xh, float *y)
{
    nd_tensor t;
    nd_cact c;
    memset(&c, 0, sizeof c);
    c.codebook = codebook;
    cq_tensor(&t, out, in, group, bits);
    nd_cq_gemv_prepared(&c, &t, blob, xh, y);
}

void ref_cq_lut2(uint32_t out, uint32_t in, uint32_t group, const void *blob, const float *codebook,
                 const float *xh, float *lut, float *y)
{
    nd_tensor t;
    nd_cact c;
    memset(&c, 0, sizeof c);
    c.codebook = codebook;
    cq_tensor(&t, out, in, group, 2);
    nd_cq_lut_build(&c, xh, nd_cq_in_pad(&t), lut);
    nd_cq_gemv_lut2(&t, blob, lut, y);
}

/* ------------------------------------------------- the whole attention() */

/* Give the hand-built model its CQ projections: per layer q, k, v, gate,
 * out_proj (2-bit, one group) as archive blobs, laid into one buffer as
 * nd_cact tensors so nd_tier_ptr / nd_cact_data resolve them, plus the gemv
 * scratch (xh, the pair table). blobs[layer*5 + t]; d_model the projections'
 * input width. Call once, after ref_session_front. */
int ref_block_setup(void *vm, uint32_t d_model, uint32_t group, const void *const *blobs,
                    const float *codebook)
{
    nd_model *m = (nd_model *)vm;
    uint32_t outs[5] = { m->n_heads * m->qk_head_dim, m->k_dim, m->v_dim, m->attn_dim, d_model };
    uint32_t ins[5] = { d_model, d_model, d_model, d_model, m->attn_dim };
    size_t total = 0, off = 0, sizes[5];
    uint32_t li, t, maxpad = 0;
    uint8_t *base;
    for (t = 0; t < 5; t++) {
        uint32_t pad = (ins[t] + group - 1) / group * group;
        sizes[t] = (size_t)outs[t] * pad / 4 + (size_t)outs[t] * (pad / group) * 2;
        if (pad > maxpad)
            maxpad = pad;
    }
    for (t = 0; t < 5; t++)
        total += sizes[t];
    total *= m->n_layers;
    base = (uint8_t *)malloc(total + 64);
    m->layer = (nd_layer *)calloc(m->n_layers, sizeof(nd_layer));
    m->xh = (float *)calloc(maxpad, sizeof(float));
    m->lut = (float *)calloc((size_t)maxpad / 2 * 16, sizeof(float));
    if (!base || !m->layer || !m->xh || !m->lut)
        return -1;
    m->c.base = base;
    m->c.size = total;
    m->c.codebook = codebook;
    for (li = 0; li < m->n_layers; li++) {
        nd_tensor *ts[5] = { &m->layer[li].q_proj, &m->layer[li].k_proj, &m->layer[li].v_proj,
                             &m->layer[li].gate_proj, &m->layer[li].out_proj };
        for (t = 0; t < 5; t++) {
            memset(ts[t], 0, sizeof *ts[t]);
            ts[t]->ndim = 2;
            ts[t]->shape[0] = outs[t];
            ts[t]->shape[1] = ins[t];
            ts[t]->group = group;
            ts[t]->bits = 2;
            ts[t]->offset = off;
            ts[t]->nbytes = sizes[t];
            memcpy(base + off, blobs[li * 5 + t], sizes[t]);
            off += sizes[t];
        }
    }
    return 0;
}

/* The engine's attention(m, li, xin, out) itself at the model's pos (the
 * rotary table of nd_model_step_hidden :2949-2954 filled first, restated),
 * with the front weights in fp16_slot[li][4..8]. */
void ref_attention_block(void *vm, uint32_t li, const float *tap_q, const float *tap_k, const float *tap_v,
                         const float *norm_q, const float *norm_k, const float *xin, float *out)
{
    nd_model *m = (nd_model *)vm;
    uint32_t i;
    for (i = 0; i < m->qk_head_dim / 2; i++) {
        float angle = (float)m->pos * m->rope_inv[i];
        m->rope_cos[i] = cosf(angle);
        m->rope_sin[i] = sinf(angle);
    }
    m->fp16_slot[li][4] = (float *)tap_q;
    m->fp16_slot[li][5] = (float *)tap_k;
    m->fp16_slot[li][6] = (float *)tap_v;
    m->fp16_slot[li][7] = (float *)norm_q;
    m->fp16_slot[li][8] = (float *)norm_k;
    attention(m, li, xin, out);
}

/* ------------------------------------------------- CPU baseline timing */

/* The batched-decode CPU baseline: n independent sessions (one per
 * sequence), each taking one store + attention() step per round, split over
 * nthreads threads by contiguous session ranges - the engine has one session
 * per model and no shared writable state on this path, so sessions run side
 * by side as separate models would. Each thread writes its own output row.
 * Returns the wall time of `rounds` rounds in seconds, CLOCK_MONOTONIC (as
 * host/nd_prof.c:45-49 times the engine). */
typedef struct {
    void **models;
    uint32_t lo, hi, li, rounds;
    const float *q, *k, *v;
    float *out;
} ref_rounds_job;

static void *ref_rounds_worker(void *arg)
{
    ref_rounds_job *j = (ref_rounds_job *)arg;
    uint32_t r, s;
    for (r = 0; r < j->rounds; r++)
        for (s = j->lo; s < j->hi; s++)
            ref_attention(j->models[s], j->li, j->q, j->k, j->v, NULL, j->out);
    return NULL;
}

double ref_attention_rounds(void **models, uint32_t n, uint32_t li, const float *q, const float *k,
                            const float *v, float *out, uint32_t out_stride, uint32_t rounds,
                            uint32_t nthreads)
{
    pthread_t th[256];
    ref_rounds_job jobs[256];
    struct timespec t0, t1;
    uint32_t t;
    if (nthreads < 1)
        nthreads = 1;
    if (nthreads > 256)
        nthreads = 256;
    if (nthreads > n)
        nthreads = n;
    for (t = 0; t < nthreads; t++) {
        jobs[t].models = models;
        jobs[t].lo = (uint32_t)((uint64_t)n * t / nthreads);
        jobs[t].hi = (uint32_t)((uint64_t)n * (t + 1) / nthreads);
        jobs[t].li = li;
        jobs[t].rounds = rounds;
        jobs[t].q = q;
        jobs[t].k = k;
        jobs[t].v = v;
        jobs[t].out = out + (size_t)t * out_stride;
    }
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (t = 1; t < nthreads; t++)
        pthread_create(&th[t], NULL, ref_rounds_worker, &jobs[t]);
    ref_rounds_worker(&jobs[0]);
    for (t = 1; t < nthreads; t++)
        pthread_join(th[t], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* ---- the engine's row seam on the host's cores ----
 *
 * nd_parallel_rows (engine/include/nd_quant.h:213-230) is the engine's only
 * parallelism: an installed splitter runs fn over disjoint row ranges at once
 * and the caller waits for all of them (the ESP32 build installs a two-core
 * one, esp32/main/main.c:191). ref_pool_start(n) installs the same contract
 * over n host threads - the caller's thread takes range 0, n - 1 persistent
 * workers the others, contiguous and as even as the row count allows, the
 * caller returning once all are done - so attention()'s own dispatch,
 * nd_parallel_rows(attn_heads, &actx, nh) (engine/src/nd_model.c:2481), runs
 * its heads on n cores. ref_pool_stop() restores the serial splitter. */
static pthread_t pool_th[256];
static int pool_n = 0, pool_quit = 0;
static uint32_t pool_gen = 0, pool_done = 0;   /* __atomic: the dispatch and its completion count */
static nd_row_fn pool_fn;
static void *pool_ctx;
static uint32_t pool_rows;
static void (*pool_saved)(nd_row_fn, void *, uint32_t);

#if defined(__x86_64__) || defined(__i386__)
#define POOL_RELAX() __builtin_ia32_pause()
#else
#define POOL_RELAX() ((void)0)
#endif

static void pool_slice(int t)
{
    uint32_t r0 = (uint32_t)((uint64_t)pool_rows * (uint32_t)t / (uint32_t)pool_n);
    uint32_t r1 = (uint32_t)((uint64_t)pool_rows * (uint32_t)(t + 1) / (uint32_t)pool_n);
    if (r0 < r1)
        pool_fn(pool_ctx, r0, r1);
}

/* Workers spin on the dispatch counter (each has a core of its own: the
 * pool is sized to the cores the process may use), so a dispatch costs a
 * cache-line handoff rather than a futex wake-up per thread. */
static void *pool_worker(void *arg)
{
    int t = (int)(intptr_t)arg;
    uint32_t seen = 0;
    for (;;) {
        uint32_t g;
        while ((g = __atomic_load_n(&pool_gen, __ATOMIC_ACQUIRE)) == seen)
            POOL_RELAX();
        seen = g;
        if (__atomic_load_n(&pool_quit, __ATOMIC_ACQUIRE))
            return NULL;
        pool_slice(t);
        __atomic_fetch_add(&pool_done, 1u, __ATOMIC_ACQ_REL);
    }
}

static void pool_split(nd_row_fn fn, void *ctx, uint32_t nrows)
{
    pool_fn = fn;
    pool_ctx = ctx;
    pool_rows = nrows;
    __atomic_store_n(&pool_done, 0u, __ATOMIC_RELAXED);
    __atomic_fetch_add(&pool_gen, 1u, __ATOMIC_RELEASE);
    pool_slice(0);
    while (__atomic_load_n(&pool_done, __ATOMIC_ACQUIRE) != (uint32_t)(pool_n - 1))
        POOL_RELAX();
}

int ref_pool_start(int n)
{
    int t;
    if (pool_n || n < 2 || n > 256)
        return -1;
    pool_n = n;
    pool_quit = 0;
    pool_gen = 0;
    for (t = 1; t < n; t++)
        if (pthread_create(&pool_th[t], NULL, pool_worker, (void *)(intptr_t)t))
            return -1;
    pool_saved = nd_parallel_rows;
    nd_parallel_rows = pool_split;
    return 0;
}

void ref_pool_stop(void)
{
    int t;
    if (!pool_n)
        return;
    nd_parallel_rows = pool_saved;
    __atomic_store_n(&pool_quit, 1, __ATOMIC_RELEASE);
    __atomic_fetch_add(&pool_gen, 1u, __ATOMIC_RELEASE);
    for (t = 1; t < pool_n; t++)
        pthread_join(pool_th[t], NULL);
    pool_n = 0;
}

/* The engine's prefill of one sequence: S tokens, each through every layer
 * (store + attention() dispatch with the heads through nd_parallel_rows, as
 * nd_model.c:2426-2483 does), pos advancing after each token
 * (esp32/main/main.c:312-315 feeds a prompt one token at a time). q/k/v hold
 * one row per token, reused by every layer; out receives the last layer's
 * rows. Wall time of the whole prefill in seconds, CLOCK_MONOTONIC. */
double ref_prefill_rounds(void *vm, uint32_t S, const float *q, const float *k, const float *v, float *out)
{
    nd_model *m = (nd_model *)vm;
    struct timespec t0, t1;
    uint32_t t, li, nh = m->n_heads, rcap = m->window - m->n_sink;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (t = 0; t < S; t++) {
        for (li = 0; li < m->n_layers; li++) {
            attn_ctx c;
            uint32_t i;
            ref_kv_store(vm, li, k + (size_t)t * m->n_kv_heads * m->qk_head_dim,
                         v + (size_t)t * m->n_kv_heads * m->v_head_dim);
            memcpy(m->q, q + (size_t)t * nh * m->qk_head_dim, sizeof(float) * nh * m->qk_head_dim);
            for (i = 0; i < nh * m->v_head_dim; i++)
                m->gate[i] = INFINITY;
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
            nd_parallel_rows(attn_heads, &c, nh);
            if (li + 1 == m->n_layers)
                memcpy(out + (size_t)t * nh * m->v_head_dim, m->attn, sizeof(float) * nh * m->v_head_dim);
        }
        m->pos++;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}
