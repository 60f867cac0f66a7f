/* nd_oracle.c - CPU restatement of the Needle attention / KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY (see nd_oracle.h): the oracle libndattn is tested
 * against, never part of the product. Must be compiled with -ffp-contract=off so that every
 * multiply and add rounds separately, as the reference's x86 host build does
 * (host/CMakeLists.txt:4-11: C99, no FMA target flags).
 */
#include "nd_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ primitives */

/* Position -> slot. Sinks keep their position; the rest ring through the
 * remaining window - n_sink slots. engine/src/nd_model.c:1302-1309. */
uint32_t ndo_kv_slot(uint32_t window, uint32_t n_sink, uint32_t p)
{
    if (p < n_sink)
        return p;
    return n_sink + (p - n_sink) % (window - n_sink);
}

/* The sink count actually pinned for a request of n: at most window-64, and
 * 0 when the window is not larger than 64. engine/src/nd_model.c:1311-1321. */
uint32_t ndo_clamp_sink(uint32_t window, uint32_t n)
{
    uint32_t cap = window > NDO_MIN_RECENT ? window - NDO_MIN_RECENT : 0u;
    return n < cap ? n : cap;
}

/* exp(x) by range reduction to 2^k * 2^f, f in [-0.5, 0.5], a degree-5
 * polynomial for 2^f and an assembled exponent field for 2^k, with saturation
 * outside +-88. Method and coefficients: engine/include/nd_quant.h:93-117. */
float ndo_expf(float x)
{
    static const float c5 = 0.0013333f, c4 = 0.0096181f, c3 = 0.0555041f,
                       c2 = 0.2402265f, c1 = 0.6931472f, c0 = 1.0f;
    float z, f, p, two_k;
    int k;
    uint32_t bits;

    if (x > 88.0f)
        return 3.4028235e38f;
    if (x < -88.0f)
        return 0.0f;
    z = x * 1.44269504f;
    k = (int)(z >= 0.0f ? z + 0.5f : z - 0.5f);   /* round half away, truncating cast */
    f = z - (float)k;
    p = c5;
    p = p * f + c4;
    p = p * f + c3;
    p = p * f + c2;
    p = p * f + c1;
    p = p * f + c0;
    bits = (uint32_t)(k + 127) << 23;
    memcpy(&two_k, &bits, sizeof two_k);
    return p * two_k;
}

/* The paired form is defined to equal two scalar calls (nd_quant.h:132-135,
 * :146-168: out-of-range pairs take the scalar path, in-range chains perform
 * the scalar operations in the scalar order). */
void ndo_expf_pair(float x0, float x1, float *r0, float *r1)
{
    *r0 = ndo_expf(x0);
    *r1 = ndo_expf(x1);
}

/* Branch on the sign so the exponential never overflows.
 * engine/src/nd_model.c:48-58 (scalar) and :96-110 (pair, same values). */
float ndo_sigmoid(float x)
{
    if (x >= 0.0f) {
        float e = ndo_expf(-x);
        return 1.0f / (1.0f + e);
    } else {
        float e = ndo_expf(x);
        return e / (1.0f + e);
    }
}

float ndo_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    float f;

    if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e == 0u) {
        f = (float)m * 5.9604644775390625e-08f;   /* m * 2^-24, exact */
        return sign ? -f : f;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, sizeof f);
    return f;
}

uint16_t ndo_f32_to_f16(float f)
{
    uint32_t x, sign, absx;
    memcpy(&x, &f, sizeof x);
    sign = (x >> 16) & 0x8000u;
    absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u)                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    if (absx >= 0x477ff000u)                       /* rounds to >= 65520: inf */
        return (uint16_t)(sign | 0x7c00u);
    if (absx < 0x38800000u) {                      /* below 2^-14: subnormal half */
        /* value / 2^-24 rounded to nearest even, computed exactly in double */
        double v = (double)fabsf(f) * 16777216.0;
        double r = nearbyint(v);                   /* default mode: ties to even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    {
        uint32_t mant = absx & 0x7fffffu, exp = (absx >> 23) - 112u;
        uint32_t h = (exp << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
            h++;
        return (uint16_t)(sign | h);
    }
}

/* ndo_f16_to_f32 of every 16-bit pattern, built once: the same values,
 * without the per-element branches. */
static float g_f16_tab[65536];
static pthread_once_t g_f16_once = PTHREAD_ONCE_INIT;

static void f16_table_init(void)
{
    uint32_t h;
    for (h = 0; h < 65536u; h++)
        g_f16_tab[h] = ndo_f16_to_f32((uint16_t)h);
}

static const float *f16_table(void)
{
    pthread_once(&g_f16_once, f16_table_init);
    return g_f16_tab;
}

/* Quotient by the residual (Markstein) form with one reciprocal: r = 1/scale,
 * y = x*r, e = fma(-scale, y, x), q = fma(e, r, y); plain x/scale for
 * |x| >= 1e30. Clamped to +-127 and rounded half-to-even by lrintf; a NaN
 * quotient (1/scale overflowing for scale < 2^-127) stores code 0, which is
 * what lrintf's out-of-range result truncates to on the x86 host build.
 * engine/src/nd_model.c:1819-1866. For normal scales this equals the IEEE
 * quotient (tests check that against the reference's own function). */
void ndo_kv_store_int8(int8_t *dst, const float *src, uint32_t n, float scale)
{
    const float r = 1.0f / scale;
    uint32_t i;
    for (i = 0; i < n; i++) {
        float x = src[i], q;
        if (x > -1e30f && x < 1e30f) {
            float e;
            q = x * r;
            e = fmaf(-scale, q, x);
            q = fmaf(e, r, q);
        } else {
            q = x / scale;
        }
        if (q != q) {
            dst[i] = 0;
            continue;
        }
        if (q > 127.0f)
            q = 127.0f;
        if (q < -127.0f)
            q = -127.0f;
        dst[i] = (int8_t)lrintf(q);
    }
}

/* scale = absmax/127, or 1 for an all-zero row. engine/src/nd_model.c:2426-2442. */
float ndo_kv_quant_row(const float *x, uint32_t n, int8_t *dst)
{
    float amax = 0.0f, scale;
    uint32_t i;
    for (i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > amax)
            amax = a;
    }
    scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    ndo_kv_store_int8(dst, x, n, scale);
    return scale;
}

/* ------------------------------------------------------------- attention */

/* Element e of a KV row as float: (float)(int8_t) for int8, exact fp16 widening
 * otherwise (nd_model.c:79-94 stages int8 this way; fp16 per the fp16 variant). */
static void stage_row(const ndo_kv_view *kv, const void *base, uint32_t slot, uint32_t g,
                      uint32_t hd, float *dst)
{
    size_t off = ((size_t)slot * kv->nkv + g) * hd;
    uint32_t i;
    if (kv->kv_dtype == NDO_KV_INT8) {
        const int8_t *r = (const int8_t *)base + off;
        for (i = 0; i < hd; i++)
            dst[i] = (float)r[i];
    } else {
        const uint16_t *r = (const uint16_t *)base + off;
        const float *tab = f16_table();
        for (i = 0; i < hd; i++)
            dst[i] = tab[r[i]];
    }
}

static float row_scale(const ndo_kv_view *kv, const float *sc, uint32_t slot, uint32_t g)
{
    return kv->kv_dtype == NDO_KV_INT8 ? sc[(size_t)slot * kv->nkv + g] : 1.0f;
}

/* Running state of one query head across the visited positions. */
typedef struct {
    float mx, denom;
    float *oh;
} head_state;

/* Score of one position, ascending pair sums: s += q[i]k[i] + q[i+1]k[i+1]:
 * the dot of a head outside a pair (the last head of an odd group,
 * nd_model.c:2259-2266). */
static float dot_pairs(const float *q, const float *k, uint32_t n)
{
    float s = 0.0f;
    uint32_t i;
    for (i = 0; i + 1u < n; i += 2u)
        s += q[i] * k[i] + q[i + 1u] * k[i + 1u];
    for (; i < n; i++)
        s += q[i] * k[i];
    return s;
}

/* The four scores of a head PAIR (A, B) over two positions (0, 1), as
 * qk_dot8 computes them (nd_model.c:2038-2083): per score, ascending pair
 * sums over whole 8-column groups, then the remaining columns one term at a
 * time (equal to dot_pairs when qk_hd is a multiple of 8). */
static void dot4_pairs8(const float *qA, const float *qB, const float *k0, const float *k1, uint32_t n,
                        float *s)
{
    float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
    uint32_t i, j;
    for (i = 0; i + 7u < n; i += 8u)
        for (j = i; j < i + 8u; j += 2u) {
            a0 += qA[j] * k0[j] + qA[j + 1u] * k0[j + 1u];
            a1 += qA[j] * k1[j] + qA[j + 1u] * k1[j + 1u];
            b0 += qB[j] * k0[j] + qB[j + 1u] * k0[j + 1u];
            b1 += qB[j] * k1[j] + qB[j + 1u] * k1[j + 1u];
        }
    for (; i < n; i++) {
        a0 += qA[i] * k0[i];
        a1 += qA[i] * k1[i];
        b0 += qB[i] * k0[i];
        b1 += qB[i] * k1[i];
    }
    s[0] = a0; s[1] = a1; s[2] = b0; s[3] = b1;
}

/* Sequential dot of the odd-tail position (nd_model.c:2319-2320). */
static float dot_seq(const float *q, const float *k, uint32_t n)
{
    float s = 0.0f;
    uint32_t i;
    for (i = 0; i < n; i++)
        s += q[i] * k[i];
    return s;
}

/* One pair step for one head: the max/rescale/exp/denominator sequence of
 * nd_model.c:2217-2249 and the P.V update of pv_pair2 (:1958-2024): rescale
 * first, then per cell the w0 term and then the w1 term, separately rounded. */
static void pair_step(head_state *h, float s0, float s1, float vs0, float vs1,
                      const float *vf0, const float *vf1, uint32_t v_hd)
{
    float mnew = s0 > s1 ? s0 : s1, w0, w1, wv0, wv1;
    uint32_t i;
    if (mnew > h->mx) {
        if (h->denom > 0.0f) {
            float r = ndo_expf(h->mx - mnew);
            h->denom *= r;
            for (i = 0; i < v_hd; i++)
                h->oh[i] *= r;
        }
        h->mx = mnew;
    }
    ndo_expf_pair(s0 - h->mx, s1 - h->mx, &w0, &w1);
    h->denom += w0 + w1;
    wv0 = w0 * vs0;
    wv1 = w1 * vs1;
    for (i = 0; i < v_hd; i++) {
        h->oh[i] += wv0 * vf0[i];
        h->oh[i] += wv1 * vf1[i];
    }
}

/* The max/rescale/exp/denominator part of a pair step for one head
 * (nd_model.c:2217-2249); returns whether oh must be rescaled by *r. */
static int pair_softmax(head_state *h, float s0, float s1, float *r, float *w0, float *w1)
{
    float mnew = s0 > s1 ? s0 : s1;
    int rs = 0;
    if (mnew > h->mx) {
        if (h->denom > 0.0f) {
            *r = ndo_expf(h->mx - mnew);
            h->denom *= *r;
            rs = 1;
        }
        h->mx = mnew;
    }
    ndo_expf_pair(s0 - h->mx, s1 - h->mx, w0, w1);
    h->denom += *w0 + *w1;
    return rs;
}

/* A pair step for two heads sharing the staged rows (pv_pair2,
 * nd_model.c:1958-2024): each head's softmax step, then one pass over the
 * cells applying each head's rescale and its w0 and w1 terms in pair_step's
 * per-cell order. */
static void pair_step2(head_state *a, head_state *b, const float *sc, float sc0, float sc1, float vs0,
                       float vs1, const float *vf0, const float *vf1, uint32_t v_hd)
{
    float ra = 1.0f, rb = 1.0f, wa0, wa1, wb0, wb1, va0, va1, vb0, vb1;
    int rsa = pair_softmax(a, sc[0] * sc0, sc[1] * sc1, &ra, &wa0, &wa1);
    int rsb = pair_softmax(b, sc[2] * sc0, sc[3] * sc1, &rb, &wb0, &wb1);
    uint32_t i;
    if (rsa)
        for (i = 0; i < v_hd; i++)
            a->oh[i] *= ra;
    if (rsb)
        for (i = 0; i < v_hd; i++)
            b->oh[i] *= rb;
    va0 = wa0 * vs0;
    va1 = wa1 * vs1;
    vb0 = wb0 * vs0;
    vb1 = wb1 * vs1;
    for (i = 0; i < v_hd; i++) {
        a->oh[i] += va0 * vf0[i];
        a->oh[i] += va1 * vf1[i];
        b->oh[i] += vb0 * vf0[i];
        b->oh[i] += vb1 * vf1[i];
    }
}

/* The single trailing position of an odd-length run (nd_model.c:2301-2340). */
static void single_step(head_state *h, float s, float vs, const float *vf, uint32_t v_hd)
{
    float w, wv;
    uint32_t i;
    if (s > h->mx) {
        if (h->denom > 0.0f) {
            float r = ndo_expf(h->mx - s);
            for (i = 0; i < v_hd; i++)
                h->oh[i] *= r;
            h->denom *= r;
        }
        h->mx = s;
    }
    w = ndo_expf(s - h->mx);
    h->denom += w;
    wv = w * vs;
    for (i = 0; i < v_hd; i++)
        h->oh[i] += wv * vf[i];
}

#define NDO_HD_MAX 256u
#define NDO_REP_MAX 64u

/* Visit one run of slots for every head of kv group g. */
static void visit_run(const ndo_kv_view *kv, uint32_t g, uint32_t rep, const float *q,
                      float scale, const uint32_t *slots, uint32_t count, head_state *hs)
{
    float kf0[NDO_HD_MAX], kf1[NDO_HD_MAX], vf0[NDO_HD_MAX], vf1[NDO_HD_MAX];
    uint32_t p, t;
    for (p = 0; p + 1u < count; p += 2u) {
        uint32_t sl0 = slots[p], sl1 = slots[p + 1u];
        float sc0 = row_scale(kv, kv->k_scale, sl0, g) * scale;
        float sc1 = row_scale(kv, kv->k_scale, sl1, g) * scale;
        float vs0 = row_scale(kv, kv->v_scale, sl0, g);
        float vs1 = row_scale(kv, kv->v_scale, sl1, g);
        stage_row(kv, kv->k, sl0, g, kv->qk_hd, kf0);
        stage_row(kv, kv->k, sl1, g, kv->qk_hd, kf1);
        stage_row(kv, kv->v, sl0, g, kv->v_hd, vf0);
        stage_row(kv, kv->v, sl1, g, kv->v_hd, vf1);
        /* heads go in pairs (t, t+1) through qk_dot8; an odd group's last
         * head takes the single-head dot (nd_model.c:2201-2266) */
        for (t = 0; t + 1u < rep; t += 2u) {
            const float *qA = q + (size_t)(g * rep + t) * kv->qk_hd;
            float sc[4];
            dot4_pairs8(qA, qA + kv->qk_hd, kf0, kf1, kv->qk_hd, sc);
            pair_step2(&hs[t], &hs[t + 1u], sc, sc0, sc1, vs0, vs1, vf0, vf1, kv->v_hd);
        }
        if (t < rep) {
            const float *qh = q + (size_t)(g * rep + t) * kv->qk_hd;
            float s0 = dot_pairs(qh, kf0, kv->qk_hd) * sc0;
            float s1 = dot_pairs(qh, kf1, kv->qk_hd) * sc1;
            pair_step(&hs[t], s0, s1, vs0, vs1, vf0, vf1, kv->v_hd);
        }
    }
    if (p < count) {
        uint32_t sl = slots[p];
        float sc = row_scale(kv, kv->k_scale, sl, g) * scale;
        float vs = row_scale(kv, kv->v_scale, sl, g);
        stage_row(kv, kv->k, sl, g, kv->qk_hd, kf0);
        stage_row(kv, kv->v, sl, g, kv->v_hd, vf0);
        for (t = 0; t < rep; t++) {
            const float *qh = q + (size_t)(g * rep + t) * kv->qk_hd;
            float s = dot_seq(qh, kf0, kv->qk_hd) * sc;
            single_step(&hs[t], s, vs, vf0, kv->v_hd);
        }
    }
}

/* Emit: out = (oh * (1/denom)) * sigmoid(gate), two roundings per element
 * (attn_gate_emit, nd_model.c:2085-2103, :2342-2357). Without a gate the
 * normalised accumulator is the output (the odd-v_hd branch, :2353-2356). */
static void emit(const head_state *h, const float *gate, float *out, uint32_t v_hd)
{
    float inv = 1.0f / h->denom;
    uint32_t i;
    for (i = 0; i < v_hd; i++) {
        float z = h->oh[i] * inv;
        out[i] = gate ? z * ndo_sigmoid(gate[i]) : z;
    }
}

void ndo_attend_runs(const ndo_kv_view *kv, const uint32_t *slots, const uint32_t *run_len,
                     uint32_t n_runs, const float *q, const float *gate, float *out)
{
    uint32_t rep = kv->nh / kv->nkv, g, t, r;
    float scale = 1.0f / sqrtf((float)kv->qk_hd);
    head_state hs[NDO_REP_MAX];

    for (g = 0; g < kv->nkv; g++) {
        const uint32_t *sl = slots;
        for (t = 0; t < rep; t++) {
            hs[t].mx = -INFINITY;
            hs[t].denom = 0.0f;
            hs[t].oh = out + (size_t)(g * rep + t) * kv->v_hd;
            memset(hs[t].oh, 0, sizeof(float) * kv->v_hd);
        }
        for (r = 0; r < n_runs; r++) {
            visit_run(kv, g, rep, q, scale, sl, run_len[r], hs);
            sl += run_len[r];
        }
        for (t = 0; t < rep; t++)
            emit(&hs[t], gate ? gate + (size_t)(g * rep + t) * kv->v_hd : NULL, hs[t].oh,
                 kv->v_hd);
    }
}

/* The dispatch arithmetic of attention(): sinks = min(n_sink, pos+1), the
 * recent run is the last min(pos+1-n_sink, window-n_sink) positions.
 * engine/src/nd_model.c:2451-2483. */
void ndo_attend(const ndo_kv_view *kv, const float *q, const float *gate, float *out)
{
    uint32_t sinks = kv->n_sink < kv->pos + 1u ? kv->n_sink : kv->pos + 1u;
    uint32_t rcap = kv->window - kv->n_sink, rfirst, rcount, i;
    uint32_t *slots = (uint32_t *)malloc(sizeof(uint32_t) * (kv->window + 1u));
    uint32_t run_len[2];

    if (kv->pos + 1u <= kv->n_sink) {
        rfirst = kv->pos + 1u;
        rcount = 0;
    } else {
        rcount = kv->pos + 1u - kv->n_sink;
        if (rcount > rcap)
            rcount = rcap;
        rfirst = kv->pos + 1u - rcount;
    }
    for (i = 0; i < sinks; i++)
        slots[i] = ndo_kv_slot(kv->window, kv->n_sink, i);
    for (i = 0; i < rcount; i++)
        slots[sinks + i] = ndo_kv_slot(kv->window, kv->n_sink, rfirst + i);
    run_len[0] = sinks;
    run_len[1] = rcount;
    ndo_attend_runs(kv, slots, run_len, 2, q, gate, out);
    free(slots);
}

void ndo_attend_f64(const ndo_kv_view *kv, const uint32_t *slots, uint32_t n_pos,
                    const float *q, const float *gate, double *out)
{
    uint32_t rep = kv->nh / kv->nkv, h, p, i;
    double scale = 1.0 / sqrt((double)kv->qk_hd);
    double *s = (double *)malloc(sizeof(double) * (n_pos ? n_pos : 1u));
    float kf[NDO_HD_MAX], vf[NDO_HD_MAX];

    for (h = 0; h < kv->nh; h++) {
        uint32_t g = h / rep;
        const float *qh = q + (size_t)h * kv->qk_hd;
        double mx = -INFINITY, den = 0.0;
        double *o = out + (size_t)h * kv->v_hd;
        for (p = 0; p < n_pos; p++) {
            double d = 0.0;
            stage_row(kv, kv->k, slots[p], g, kv->qk_hd, kf);
            for (i = 0; i < kv->qk_hd; i++)
                d += (double)qh[i] * (double)kf[i];
            s[p] = d * (double)row_scale(kv, kv->k_scale, slots[p], g) * scale;
            if (s[p] > mx)
                mx = s[p];
        }
        for (i = 0; i < kv->v_hd; i++)
            o[i] = 0.0;
        for (p = 0; p < n_pos; p++) {
            double w = exp(s[p] - mx);
            double vs = (double)row_scale(kv, kv->v_scale, slots[p], g);
            den += w;
            stage_row(kv, kv->v, slots[p], g, kv->v_hd, vf);
            for (i = 0; i < kv->v_hd; i++)
                o[i] += w * vs * (double)vf[i];
        }
        for (i = 0; i < kv->v_hd; i++) {
            double gt = gate ? 1.0 / (1.0 + exp(-(double)gate[(size_t)h * kv->v_hd + i])) : 1.0;
            o[i] = o[i] / den * gt;
        }
    }
    free(s);
}

/* --------------------------------------------------------------- session */

static size_t elem_size(int dt) { return dt == NDO_KV_INT8 ? 1u : 2u; }

int ndo_session_init(ndo_session *s, uint32_t n_layers, uint32_t nh, uint32_t nkv,
                     uint32_t qk_hd, uint32_t v_hd, uint32_t window, int kv_dtype)
{
    size_t slots = (size_t)n_layers * window;
    memset(s, 0, sizeof *s);
    if (!n_layers || !nh || !nkv || nh % nkv || nh / nkv > NDO_REP_MAX || !qk_hd ||
        !v_hd || qk_hd > NDO_HD_MAX || v_hd > NDO_HD_MAX || !window)
        return -1;
    s->n_layers = n_layers; s->nh = nh; s->nkv = nkv;
    s->qk_hd = qk_hd; s->v_hd = v_hd; s->window = window; s->kv_dtype = kv_dtype;
    s->k_cache = calloc(slots * nkv * qk_hd, elem_size(kv_dtype));
    s->v_cache = calloc(slots * nkv * v_hd, elem_size(kv_dtype));
    s->k_scale = (float *)calloc(slots * nkv, sizeof(float));
    s->v_scale = (float *)calloc(slots * nkv, sizeof(float));
    if (!s->k_cache || !s->v_cache || !s->k_scale || !s->v_scale) {
        ndo_session_free(s);
        return -2;
    }
    return 0;
}

void ndo_session_free(ndo_session *s)
{
    free(s->k_cache); free(s->v_cache); free(s->k_scale); free(s->v_scale);
    free(s->q_hist); free(s->k_hist); free(s->v_hist);
    free(s->snap_q_hist); free(s->snap_k_hist); free(s->snap_v_hist);
    free(s->rope_inv);
    memset(s, 0, sizeof *s);
}

/* Floats in one of the three history arrays over all layers. */
static size_t hist_len(const ndo_session *s, int which)
{
    size_t dim = which == 0 ? (size_t)s->nh * s->qk_hd
               : which == 1 ? (size_t)s->nkv * s->qk_hd : (size_t)s->nkv * s->v_hd;
    return (size_t)s->n_layers * s->taps * dim;
}

/* The histories take part in reset / snapshot / rewind as in
 * nd_model.c:1423-1425, :1451-1453, :1575-1580. */
static void hist_move(ndo_session *s, int to_snap)
{
    float *live[3] = { s->q_hist, s->k_hist, s->v_hist };
    float *snap[3] = { s->snap_q_hist, s->snap_k_hist, s->snap_v_hist };
    int a;
    if (!s->taps)
        return;
    for (a = 0; a < 3; a++) {
        if (to_snap)
            memcpy(snap[a], live[a], sizeof(float) * hist_len(s, a));
        else
            memcpy(live[a], snap[a], sizeof(float) * hist_len(s, a));
    }
}

void ndo_reset(ndo_session *s)
{
    s->pos = 0;
    s->n_sink = 0;
    s->has_snap = 0;
    if (s->taps) {
        memset(s->q_hist, 0, sizeof(float) * hist_len(s, 0));
        memset(s->k_hist, 0, sizeof(float) * hist_len(s, 1));
        memset(s->v_hist, 0, sizeof(float) * hist_len(s, 2));
    }
}

void ndo_set_sink(ndo_session *s, uint32_t n)
{
    s->n_sink = ndo_clamp_sink(s->window, n);
}

int ndo_snapshot(ndo_session *s)
{
    ndo_set_sink(s, s->pos);
    s->snap_pos = s->pos;
    hist_move(s, 1);
    s->has_snap = 1;
    return 0;
}

void ndo_rewind(ndo_session *s)
{
    if (!s->has_snap) {
        ndo_reset(s);
        return;
    }
    s->pos = s->snap_pos;
    hist_move(s, 0);
}

struct ndo_prefix {
    const ndo_session *owner;
    uint32_t pos, sink, live;
    unsigned char data[];
};

/* The live slots [0, min(snap_pos+1, window)) of every layer's K, V and
 * scales, in that order (prefix_kv / prefix_copy, nd_model.c:1466-1529). */
static size_t prefix_bytes(const ndo_session *s, uint32_t live)
{
    size_t es = elem_size(s->kv_dtype), per_layer;
    per_layer = (size_t)live * s->nkv * ((s->qk_hd + s->v_hd) * es + 2u * sizeof(float));
    return per_layer * s->n_layers + sizeof(float) * (hist_len(s, 0) + hist_len(s, 1) + hist_len(s, 2));
}

static void prefix_move(ndo_session *s, unsigned char *data, uint32_t live, int restore)
{
    size_t es = elem_size(s->kv_dtype);
    size_t rows[4], strides[4];
    unsigned char *bases[4];
    uint32_t a, l;
    size_t off = 0;

    rows[0] = (size_t)s->nkv * s->qk_hd * es;  bases[0] = (unsigned char *)s->k_cache;
    rows[1] = (size_t)s->nkv * s->v_hd * es;   bases[1] = (unsigned char *)s->v_cache;
    rows[2] = (size_t)s->nkv * sizeof(float);  bases[2] = (unsigned char *)s->k_scale;
    rows[3] = (size_t)s->nkv * sizeof(float);  bases[3] = (unsigned char *)s->v_scale;
    for (a = 0; a < 4; a++) {
        strides[a] = rows[a] * s->window;
        for (l = 0; l < s->n_layers; l++) {
            unsigned char *r = bases[a] + (size_t)l * strides[a];
            size_t n = rows[a] * live;
            if (restore)
                memcpy(r, data + off, n);
            else
                memcpy(data + off, r, n);
            off += n;
        }
    }
    /* then the snapshot histories (prefix_copy, nd_model.c:1519-1521) */
    {
        float *snap[3] = { s->snap_q_hist, s->snap_k_hist, s->snap_v_hist };
        for (a = 0; a < 3 && s->taps; a++) {
            size_t n = sizeof(float) * hist_len(s, (int)a);
            if (restore)
                memcpy(snap[a], data + off, n);
            else
                memcpy(data + off, snap[a], n);
            off += n;
        }
    }
}

ndo_prefix *ndo_prefix_save(ndo_session *s)
{
    uint32_t live;
    ndo_prefix *p;
    if (!s->has_snap || s->pos != s->snap_pos)
        return NULL;
    live = s->snap_pos + 1u < s->window ? s->snap_pos + 1u : s->window;
    p = (ndo_prefix *)malloc(sizeof *p + prefix_bytes(s, live));
    if (!p)
        return NULL;
    p->owner = s;
    p->pos = s->snap_pos;
    p->sink = s->n_sink;
    p->live = live;
    prefix_move(s, p->data, live, 0);
    return p;
}

int ndo_prefix_restore(ndo_session *s, const ndo_prefix *p)
{
    if (!p || p->owner != s)
        return -1;
    s->snap_pos = p->pos;
    s->n_sink = p->sink;
    prefix_move(s, (unsigned char *)p->data, p->live, 1);
    s->has_snap = 1;
    ndo_rewind(s);
    return 0;
}

void ndo_prefix_free(ndo_prefix *p) { free(p); }

void ndo_view(const ndo_session *s, uint32_t li, ndo_kv_view *kv)
{
    size_t es = elem_size(s->kv_dtype);
    size_t slots = (size_t)li * s->window;
    kv->nh = s->nh; kv->nkv = s->nkv; kv->qk_hd = s->qk_hd; kv->v_hd = s->v_hd;
    kv->window = s->window; kv->n_sink = s->n_sink; kv->pos = s->pos;
    kv->kv_dtype = s->kv_dtype;
    kv->k = (const unsigned char *)s->k_cache + slots * s->nkv * s->qk_hd * es;
    kv->v = (const unsigned char *)s->v_cache + slots * s->nkv * s->v_hd * es;
    kv->k_scale = s->k_scale + slots * s->nkv;
    kv->v_scale = s->v_scale + slots * s->nkv;
}

void ndo_kv_store(ndo_session *s, uint32_t li, const float *k, const float *v)
{
    uint32_t slot = ndo_kv_slot(s->window, s->n_sink, s->pos), g, i;
    size_t row = (size_t)li * s->window + slot;
    for (g = 0; g < s->nkv; g++) {
        const float *kr = k + (size_t)g * s->qk_hd, *vr = v + (size_t)g * s->v_hd;
        size_t ko = (row * s->nkv + g) * s->qk_hd, vo = (row * s->nkv + g) * s->v_hd;
        if (s->kv_dtype == NDO_KV_INT8) {
            s->k_scale[row * s->nkv + g] = ndo_kv_quant_row(kr, s->qk_hd, (int8_t *)s->k_cache + ko);
            s->v_scale[row * s->nkv + g] = ndo_kv_quant_row(vr, s->v_hd, (int8_t *)s->v_cache + vo);
        } else {
            uint16_t *kd = (uint16_t *)s->k_cache + ko, *vd = (uint16_t *)s->v_cache + vo;
            for (i = 0; i < s->qk_hd; i++)
                kd[i] = ndo_f32_to_f16(kr[i]);
            for (i = 0; i < s->v_hd; i++)
                vd[i] = ndo_f32_to_f16(vr[i]);
            s->k_scale[row * s->nkv + g] = 1.0f;
            s->v_scale[row * s->nkv + g] = 1.0f;
        }
    }
}

void ndo_attend_session(const ndo_session *s, uint32_t li, const float *q,
                        const float *gate, float *out)
{
    ndo_kv_view kv;
    ndo_view(s, li, &kv);
    ndo_attend(&kv, q, gate, out);
}

void ndo_attention(ndo_session *s, uint32_t li, const float *q, const float *k,
                   const float *v, const float *gate, float *out)
{
    ndo_kv_store(s, li, k, v);
    ndo_attend_session(s, li, q, gate, out);
}

void ndo_step_end(ndo_session *s) { s->pos++; }

void ndo_prefill_tokens(ndo_session *s, uint32_t li, uint32_t n, const float *q,
                        const float *k, const float *v, const float *gate, float *out)
{
    uint32_t p0 = s->pos, t;
    for (t = 0; t < n; t++) {
        s->pos = p0 + t;
        ndo_attention(s, li, q + (size_t)t * s->nh * s->qk_hd, k + (size_t)t * s->nkv * s->qk_hd,
                      v + (size_t)t * s->nkv * s->v_hd,
                      gate ? gate + (size_t)t * s->nh * s->v_hd : NULL,
                      out + (size_t)t * s->nh * s->v_hd);
    }
    s->pos = p0;
}

/* --------------------------------------------------------- attention front */

void ndo_rope_inv(float theta, uint32_t qk_hd, float *inv)
{
    uint32_t i;
    for (i = 0; i < qk_hd / 2; i++)
        inv[i] = 1.0f / powf(theta, (float)(2 * i) / (float)qk_hd);
}

void ndo_rope_row(const float *inv, uint32_t qk_hd, uint32_t pos, float *cs, float *sn)
{
    uint32_t i;
    for (i = 0; i < qk_hd / 2; i++) {
        float angle = (float)pos * inv[i];
        cs[i] = cosf(angle);
        sn[i] = sinf(angle);
    }
}

void ndo_tap_conv(float *proj, float *hist, const float *w, uint32_t taps, uint32_t pos,
                  uint32_t dim)
{
    uint32_t nt = taps <= pos + 1u ? taps : pos + 1u, i, j;
    memcpy(hist + (size_t)(pos % taps) * dim, proj, sizeof(float) * dim);
    for (i = 0; i < dim; i++) {
        float acc = 0.0f;
        for (j = 0; j < nt; j++)
            acc += w[(size_t)j * dim + i] * hist[(size_t)((pos - j) % taps) * dim + i];
        proj[i] = acc;
    }
}

void ndo_zcrms_heads(float *x, uint32_t nheads, uint32_t dim, const float *s, const float *cs,
                     const float *sn)
{
    uint32_t h, i, half = dim / 2;
    for (h = 0; h < nheads; h++) {
        float *r = x + (size_t)h * dim;
        float ss = 0.0f, inv;
        for (i = 0; i < dim; i++)
            ss += r[i] * r[i];
        inv = 1.0f / sqrtf(ss / (float)dim + 1e-6f);      /* ND_EPS, nd_model.c:31 */
        for (i = 0; i < half; i++) {
            float a = (1.0f + s[i]) * r[i] * inv;
            float b = (1.0f + s[i + half]) * r[i + half] * inv;
            r[i] = a * cs[i] - b * sn[i];
            r[i + half] = b * cs[i] + a * sn[i];
        }
        if (2u * half < dim)
            r[dim - 1] = (1.0f + s[dim - 1]) * r[dim - 1] * inv;
    }
}

int ndo_session_front(ndo_session *s, uint32_t taps, float rope_theta)
{
    int a;
    float **live[3] = { &s->q_hist, &s->k_hist, &s->v_hist };
    float **snap[3] = { &s->snap_q_hist, &s->snap_k_hist, &s->snap_v_hist };
    if (!taps || s->taps)
        return -1;
    s->taps = taps;
    for (a = 0; a < 3; a++) {
        *live[a] = (float *)calloc(hist_len(s, a), sizeof(float));
        *snap[a] = (float *)calloc(hist_len(s, a), sizeof(float));
        if (!*live[a] || !*snap[a])
            return -2;
    }
    s->rope_inv = (float *)malloc(sizeof(float) * (s->qk_hd / 2 + 1));
    if (!s->rope_inv)
        return -2;
    ndo_rope_inv(rope_theta, s->qk_hd, s->rope_inv);
    return 0;
}

void ndo_front(ndo_session *s, uint32_t li, const ndo_front_w *w, float *q, float *k, float *v)
{
    uint32_t dq = s->nh * s->qk_hd, dk = s->nkv * s->qk_hd, dv = s->nkv * s->v_hd;
    float cs[NDO_HD_MAX / 2], sn[NDO_HD_MAX / 2];
    ndo_rope_row(s->rope_inv, s->qk_hd, s->pos, cs, sn);
    ndo_tap_conv(q, s->q_hist + (size_t)li * s->taps * dq, w->tap_q, s->taps, s->pos, dq);
    ndo_tap_conv(k, s->k_hist + (size_t)li * s->taps * dk, w->tap_k, s->taps, s->pos, dk);
    ndo_tap_conv(v, s->v_hist + (size_t)li * s->taps * dv, w->tap_v, s->taps, s->pos, dv);
    ndo_zcrms_heads(q, s->nh, s->qk_hd, w->norm_q, cs, sn);
    ndo_zcrms_heads(k, s->nkv, s->qk_hd, w->norm_k, cs, sn);
}

/* --------------------------------------------------------- CQ projections */

uint32_t ndo_cq_in_pad(uint32_t in, uint32_t group) { return (in + group - 1) / group * group; }

void ndo_fwht(float *x, uint32_t n)
{
    uint32_t len, i, j;
    for (len = 1; len < n; len <<= 1)
        for (i = 0; i < n; i += len << 1)
            for (j = i; j < i + len; j++) {
                float a = x[j], b = x[j + len];
                x[j] = a + b;
                x[j + len] = a - b;
            }
}

void ndo_cq_prepare(uint32_t in, uint32_t group, const float *x, float *xh)
{
    uint32_t in_pad = ndo_cq_in_pad(in, group), gi, j;
    float scale = 1.0f / sqrtf((float)group);
    memcpy(xh, x, sizeof(float) * in);
    memset(xh + in, 0, sizeof(float) * (in_pad - in));
    for (gi = 0; gi < in_pad / group; gi++) {
        float *blk = xh + (size_t)gi * group;
        ndo_fwht(blk, group);
        for (j = 0; j < group; j++)
            blk[j] = blk[j] * scale;
    }
}

static uint32_t load_u32le(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* One group's sum of cb[idx] * xh: four interleaved accumulators for the
 * byte-aligned 2- and 4-bit packings, one running sum otherwise. */
static float cq_dot_group(const uint8_t *p, uint32_t bit_off, uint32_t bits, uint32_t g,
                          const float *cb, const float *xh)
{
    float s = 0.0f, s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    uint32_t j, k;
    if ((bits == 2 || bits == 4) && (bit_off & 7u) == 0) {
        const uint8_t *q = p + (bit_off >> 3);
        const uint32_t per = 32 / bits, mask = (1u << bits) - 1u;   /* weights per word */
        for (j = 0; j < g; j += per) {
            uint32_t w = load_u32le(q);
            q += 4;
            for (k = 0; k < per; k++) {
                float t = cb[(w >> (k * bits)) & mask] * xh[j + k];
                switch (k & 3u) {
                case 0: s0 += t; break;
                case 1: s1 += t; break;
                case 2: s2 += t; break;
                default: s3 += t; break;
                }
            }
        }
        return (s0 + s1) + (s2 + s3);
    }
    for (j = 0; j < g; j++) {
        uint32_t b = bit_off + j * bits, byt = b >> 3, sh = b & 7u, w = p[byt];
        if (sh + bits > 8)
            w |= (uint32_t)p[byt + 1] << 8;
        s += cb[(w >> sh) & ((1u << bits) - 1u)] * xh[j];
    }
    return s;
}

void ndo_cq_gemv(uint32_t out, uint32_t in, uint32_t group, uint32_t bits, const void *blob,
                 const float *cb, const float *xh, float *y)
{
    uint32_t in_pad = ndo_cq_in_pad(in, group), ngroup = in_pad / group;
    size_t rowbytes = (size_t)in_pad * bits / 8;
    const uint8_t *packed = (const uint8_t *)blob;
    const uint8_t *nb = packed + (size_t)out * rowbytes;     /* fp16 norms [out][ngroup] */
    uint32_t r, gi;
    for (r = 0; r < out; r++) {
        float acc = 0.0f;
        for (gi = 0; gi < ngroup; gi++) {
            size_t o = ((size_t)r * ngroup + gi) * 2;
            float nf = ndo_f16_to_f32((uint16_t)(nb[o] | (nb[o + 1] << 8)));
            acc += nf * cq_dot_group(packed + (size_t)r * rowbytes, gi * group * bits, bits, group, cb,
                                     xh + (size_t)gi * group);
        }
        y[r] = acc;
    }
}

void ndo_cq_lut_build(const float *cb, const float *xh, uint32_t in_pad, float *lut)
{
    uint32_t p, i0, i1;
    for (p = 0; p < in_pad / 2; p++) {
        float a[4], b[4];
        for (i0 = 0; i0 < 4; i0++) {
            a[i0] = cb[i0] * xh[2 * p];
            b[i0] = cb[i0] * xh[2 * p + 1];
        }
        for (i1 = 0; i1 < 4; i1++)
            for (i0 = 0; i0 < 4; i0++)
                lut[(size_t)p * 16 + i0 + 4 * i1] = a[i0] + b[i1];
    }
}

void ndo_cq_gemv_lut2(uint32_t out, uint32_t in, uint32_t group, const void *blob,
                      const float *lut, float *y)
{
    uint32_t in_pad = ndo_cq_in_pad(in, group), ngroup = in_pad / group;
    size_t rowbytes = (size_t)in_pad / 4;
    const uint8_t *packed = (const uint8_t *)blob;
    const uint8_t *nb = packed + (size_t)out * rowbytes;
    uint32_t r, gi, j, k;
    for (r = 0; r < out; r++) {
        float acc = 0.0f;
        for (gi = 0; gi < ngroup; gi++) {
            size_t o = ((size_t)r * ngroup + gi) * 2;
            float nf = ndo_f16_to_f32((uint16_t)(nb[o] | (nb[o + 1] << 8)));
            float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const uint8_t *q = packed + (size_t)r * rowbytes + (size_t)gi * group / 4;
            const float *T = lut + (size_t)gi * (group / 2) * 16;
            /* one word = 8 pairs; pair k of the word indexes table block k */
            for (j = 0; j < group; j += 16) {
                uint32_t w = load_u32le(q);
                q += 4;
                for (k = 0; k < 8; k++)
                    s[k & 3u] += T[16 * k + ((w >> (4 * k)) & 15u)];
                T += 128;
            }
            acc += nf * ((s[0] + s[1]) + (s[2] + s[3]));
        }
        y[r] = acc;
    }
}

/* ------------------------------------------------ the whole attention block */

int ndo_attention_block(ndo_session *s, uint32_t li, const ndo_front_w *fw, const ndo_block_w *bw,
                        const float *xin, float *out)
{
    uint32_t dq = s->nh * s->qk_hd, dk = s->nkv * s->qk_hd, dv = s->nkv * s->v_hd, da = s->nh * s->v_hd;
    uint32_t pin = ndo_cq_in_pad(bw->d_model, bw->group), pat = ndo_cq_in_pad(da, bw->group);
    uint32_t pmax = pin > pat ? pin : pat;
    float *xh = (float *)malloc(sizeof(float) * pmax);
    float *lut = (float *)malloc(sizeof(float) * (pmax / 2) * 16);
    float *q = (float *)malloc(sizeof(float) * dq), *k = (float *)malloc(sizeof(float) * dk);
    float *v = (float *)malloc(sizeof(float) * dv), *g = (float *)malloc(sizeof(float) * da);
    float *att = (float *)malloc(sizeof(float) * da);
    int rc = -2;
    if (!s->taps)
        rc = -1;
    else if (xh && lut && q && k && v && g && att) {
        ndo_cq_prepare(bw->d_model, bw->group, xin, xh);
        ndo_cq_lut_build(bw->cb2, xh, pin, lut);
        ndo_cq_gemv_lut2(dq, bw->d_model, bw->group, bw->blob[0], lut, q);
        ndo_cq_gemv_lut2(dk, bw->d_model, bw->group, bw->blob[1], lut, k);
        ndo_cq_gemv_lut2(dv, bw->d_model, bw->group, bw->blob[2], lut, v);
        ndo_cq_gemv_lut2(da, bw->d_model, bw->group, bw->blob[3], lut, g);
        ndo_front(s, li, fw, q, k, v);
        ndo_attention(s, li, q, k, v, g, att);
        ndo_cq_prepare(da, bw->group, att, xh);
        ndo_cq_lut_build(bw->cb2, xh, pat, lut);
        ndo_cq_gemv_lut2(bw->d_model, da, bw->group, bw->blob[4], lut, out);
        rc = 0;
    }
    free(xh); free(lut); free(q); free(k); free(v); free(g); free(att);
    return rc;
}

/* ------------------------------------------------------ threaded baseline */

typedef struct {
    const ndo_batch_f16 *b;
    uint32_t s0, s1;
} batch_job;

static void decode_one(const ndo_batch_f16 *b, uint32_t s)
{
    ndo_kv_view kv;
    uint32_t L = b->len[s], g, i;
    uint16_t *kc = b->kbase + b->koff[s], *vc = b->vbase + b->voff[s];
    const float *kn = b->k_new + (size_t)s * b->nkv * b->qk_hd;
    const float *vn = b->v_new + (size_t)s * b->nkv * b->v_hd;

    /* store the new token at slot L-1, then attend over [0, L) */
    for (g = 0; g < b->nkv; g++) {
        for (i = 0; i < b->qk_hd; i++)
            kc[((size_t)(L - 1u) * b->nkv + g) * b->qk_hd + i] = ndo_f32_to_f16(kn[g * b->qk_hd + i]);
        for (i = 0; i < b->v_hd; i++)
            vc[((size_t)(L - 1u) * b->nkv + g) * b->v_hd + i] = ndo_f32_to_f16(vn[g * b->v_hd + i]);
    }
    kv.nh = b->nh; kv.nkv = b->nkv; kv.qk_hd = b->qk_hd; kv.v_hd = b->v_hd;
    kv.window = L; kv.n_sink = 0; kv.pos = L - 1u; kv.kv_dtype = NDO_KV_F16;
    kv.k = kc; kv.v = vc; kv.k_scale = NULL; kv.v_scale = NULL;
    ndo_attend(&kv, b->q + (size_t)s * b->nh * b->qk_hd,
               b->gate ? b->gate + (size_t)s * b->nh * b->v_hd : NULL,
               b->out + (size_t)s * b->nh * b->v_hd);
}

static void *batch_worker(void *arg)
{
    batch_job *j = (batch_job *)arg;
    uint32_t s;
    for (s = j->s0; s < j->s1; s++)
        decode_one(j->b, s);
    return NULL;
}

int ndo_decode_batch_f16(const ndo_batch_f16 *b, int nthreads)
{
    pthread_t th[256];
    batch_job jobs[256];
    int t, started = 0;
    if (nthreads < 1)
        nthreads = 1;
    if (nthreads > 256)
        nthreads = 256;
    for (t = 0; t < nthreads; t++) {
        jobs[t].b = b;
        jobs[t].s0 = (uint32_t)((uint64_t)b->nseq * t / nthreads);
        jobs[t].s1 = (uint32_t)((uint64_t)b->nseq * (t + 1) / nthreads);
    }
    if (nthreads == 1) {
        batch_worker(&jobs[0]);
        return 0;
    }
    for (t = 0; t < nthreads; t++) {
        if (pthread_create(&th[t], NULL, batch_worker, &jobs[t]) != 0)
            break;
        started++;
    }
    for (t = started; t < nthreads; t++)      /* run what could not be spawned */
        batch_worker(&jobs[t]);
    for (t = 0; t < started; t++)
        pthread_join(th[t], NULL);
    return 0;
}
