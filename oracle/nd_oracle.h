/* nd_oracle.h - CPU restatement of the Needle engine's attention / KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the oracle the HIP library is compared
 * against; only tests/, the package smoke check and bench.py's cpu_baseline leg
 * may load it. The product (libndattn) never links or calls it.
 *
 * Every function restates the behaviour of the reference engine
 * (iammrduncan/esp32-needle-3) in code written for this project; each cites the
 * reference file:line it follows. Floating-point evaluation order matches the
 * reference statement for statement (build with -ffp-contract=off), so on the
 * int8 path the outputs are bit-identical to the reference's host build. That
 * claim is pinned by tests against a harness compiled from the reference's own
 * sources (oracle/ref_harness.c), not by reading this file.
 *
 * Pinning status per function:
 *   ndo_kv_slot, ndo_clamp_sink           - pinned: reference harness + brute force
 *   ndo_expf, ndo_expf_pair, ndo_sigmoid  - pinned: reference harness + exp_pairs fixture + libm bound
 *   ndo_kv_quant_row                      - pinned: reference harness (bit-exact), closed form
 *   ndo_attend (int8)                     - pinned: reference harness (bit-exact), float64 textbook
 *   ndo_attend (fp16)                     - pinned: float64 textbook + special cases (the reference
 *                                           has no fp16 KV path)
 *   session/prefix functions              - pinned: reference harness session replay
 *   ndo_tap_conv, ndo_zcrms_heads,
 *   ndo_front (+ its session state)       - pinned: reference harness (bit-exact tap_projection,
 *                                           zcrms_heads, snapshot/rewind/prefix of the histories)
 *   ndo_fwht, ndo_cq_prepare, ndo_cq_gemv,
 *   ndo_cq_lut_build, ndo_cq_gemv_lut2    - pinned: reference harness (bit-exact nd_fwht,
 *                                           nd_cq_prepare, nd_cq_gemv_prepared, nd_cq_lut_build,
 *                                           nd_cq_gemv_lut2) + float64 dequantised matvec
 *   ndo_attention_block                   - pinned: reference harness (bit-exact against the
 *                                           engine's own attention() over sessions)
 *   ndo_rope_inv, ndo_rope_row            - pinned: float64 bound (<= 1 ulp of the exact value
 *                                           of the rounded argument); the reference computes
 *                                           them inline in nd_model_open / step_hidden, so no
 *                                           harness can call them
 */
#ifndef ND_ORACLE_H
#define ND_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Recent slots kept free by the sink clamp (nd_model.c:1311-1312). */
#define NDO_MIN_RECENT 64u

enum { NDO_KV_INT8 = 0, NDO_KV_F16 = 1 };

/* ---- scalar primitives ---- */
uint32_t ndo_kv_slot(uint32_t window, uint32_t n_sink, uint32_t p);
uint32_t ndo_clamp_sink(uint32_t window, uint32_t n);
float    ndo_expf(float x);
void     ndo_expf_pair(float x0, float x1, float *r0, float *r1);
float    ndo_sigmoid(float x);
float    ndo_f16_to_f32(uint16_t h);
uint16_t ndo_f32_to_f16(float f);                 /* round to nearest even */

/* Per-(slot, kv-head) symmetric int8 row quantisation: returns the scale and
 * writes n codes. nd_model.c:2426-2449 (absmax, scale) + :1819-1866 (store). */
float    ndo_kv_quant_row(const float *x, uint32_t n, int8_t *dst);
/* The store alone, for a given scale (nd_model.c:1819-1866). */
void     ndo_kv_store_int8(int8_t *dst, const float *src, uint32_t n, float scale);

/* ---- one layer's attention over an explicit KV view ----
 *
 * The KV view is the engine's per-layer slot array: slot s of kv-head g holds
 * k at k + (s*nkv + g)*qk_hd (int8 or fp16 by kv_dtype), its scale at
 * k_scale[s*nkv + g] (int8 only), and likewise for v. */
typedef struct {
    uint32_t nh, nkv, qk_hd, v_hd, window, n_sink, pos;
    int      kv_dtype;
    const void  *k, *v;
    const float *k_scale, *v_scale;
} ndo_kv_view;

/* attn_heads for all query heads + the attention() dispatch arithmetic
 * (nd_model.c:2105-2359, :2451-2483). q [nh*qk_hd], gate [nh*v_hd] or NULL
 * (NULL: no output gate), out [nh*v_hd]. */
void ndo_attend(const ndo_kv_view *kv, const float *q, const float *gate, float *out);

/* Same, over an explicit position list instead of the sink/ring runs: every
 * listed slot is visited in order, pairs restarting at each run boundary given
 * in run_len[] (sum = n_pos). Used for the shared-prefix layout checks. */
void ndo_attend_runs(const ndo_kv_view *kv, const uint32_t *slots, const uint32_t *run_len,
                     uint32_t n_runs, const float *q, const float *gate, float *out);

/* Float64 textbook attention over the same (dequantised) KV, positions listed
 * explicitly: out = softmax(q.k * scale_k / sqrt(qk_hd)) . (v * scale_v) * sigmoid(gate). */
void ndo_attend_f64(const ndo_kv_view *kv, const uint32_t *slots, uint32_t n_pos,
                    const float *q, const float *gate, double *out);

/* ---- session: the engine's KV state for one sequence (nd_model.h:132-148) ---- */
typedef struct {
    uint32_t n_layers, nh, nkv, qk_hd, v_hd, window;
    int      kv_dtype;
    uint32_t pos, n_sink;
    int      has_snap;
    uint32_t snap_pos;
    void    *k_cache, *v_cache;       /* [layer][window][nkv*hd] int8 or fp16 */
    float   *k_scale, *v_scale;       /* [layer][window][nkv] (int8 only)   */
    /* attention front state (ndo_session_front): tap histories of the raw
     * projections [layer][tap][dim] (nd_model.h:147,167) and the rotary
     * inverse frequencies [qk_hd/2] (nd_model.h:170). taps = 0: no front. */
    uint32_t taps;
    float   *q_hist, *k_hist, *v_hist;
    float   *snap_q_hist, *snap_k_hist, *snap_v_hist;
    float   *rope_inv;
} ndo_session;

int  ndo_session_init(ndo_session *s, uint32_t n_layers, uint32_t nh, uint32_t nkv,
                      uint32_t qk_hd, uint32_t v_hd, uint32_t window, int kv_dtype);
void ndo_session_free(ndo_session *s);
void ndo_reset(ndo_session *s);                      /* nd_model.c:1557-1581 (KV part) */
void ndo_set_sink(ndo_session *s, uint32_t n);       /* nd_model.c:1314-1321 */
int  ndo_snapshot(ndo_session *s);                   /* nd_model.c:1395-1434 (KV part) */
void ndo_rewind(ndo_session *s);                     /* nd_model.c:1436-1460 */

typedef struct ndo_prefix ndo_prefix;
ndo_prefix *ndo_prefix_save(ndo_session *s);        /* nd_model.c:1531-1541 */
int  ndo_prefix_restore(ndo_session *s, const ndo_prefix *p); /* nd_model.c:1543-1553 */
void ndo_prefix_free(ndo_prefix *p);

/* Store this position's K/V for layer li (k [nkv*qk_hd], v [nkv*v_hd] fp32;
 * int8: quantised per kv-head, fp16: rounded to nearest even) and attend.
 * nd_model.c:2426-2483. Does not advance pos. */
void ndo_attention(ndo_session *s, uint32_t li, const float *q, const float *k,
                   const float *v, const float *gate, float *out);
void ndo_kv_store(ndo_session *s, uint32_t li, const float *k, const float *v);
void ndo_attend_session(const ndo_session *s, uint32_t li, const float *q,
                        const float *gate, float *out);
void ndo_step_end(ndo_session *s);                   /* pos++ (nd_model.c:3094) */
void ndo_view(const ndo_session *s, uint32_t li, ndo_kv_view *kv);

/* ---- attention front: qkv tap convolution, per-head ZC-RMSNorm + RoPE ----
 *
 * What attention() does to the raw q/k/v projections before the KV store
 * (nd_model.c:2413-2424): a causal depthwise convolution over the last `taps`
 * raw projections of each column, then for q and k a per-head RMS norm with a
 * (1 + s) scale shared by all heads, fused with GPT-NeoX half-split rotary
 * embedding at the current position. v gets the convolution only. */

/* rope_inv[i] = 1 / theta^(2i/qk_hd), i < qk_hd/2 (nd_model.c:1233-1236). */
void ndo_rope_inv(float theta, uint32_t qk_hd, float *inv);
/* cos/sin of pos * rope_inv[i] for one position (nd_model.c:2949-2954). */
void ndo_rope_row(const float *inv, uint32_t qk_hd, uint32_t pos, float *cs, float *sn);
/* One projection's tap convolution at position pos (tap_projection + tap_rows,
 * nd_model.c:2361-2379, :1748-1802): hist [taps][dim] of this layer receives
 * proj in slot pos % taps, then proj[i] = sum over j < min(taps, pos+1), in
 * ascending j from +0, of w[j][i] * hist[(pos - j) % taps][i]. */
void ndo_tap_conv(float *proj, float *hist, const float *w, uint32_t taps, uint32_t pos,
                  uint32_t dim);
/* In-place per-head ZC-RMSNorm with the rotary emit folded in
 * (zcrms_head_rows, nd_model.c:324-360): x [nheads][dim], s [dim],
 * cs/sn [dim/2]. */
void ndo_zcrms_heads(float *x, uint32_t nheads, uint32_t dim, const float *s, const float *cs,
                     const float *sn);

/* One layer's front weights: the staged fp32 tap weights [taps][dim] for q
 * (dim nh*qk_hd), k (nkv*qk_hd), v (nkv*v_hd) and the q/k norm scales [qk_hd]
 * (the engine's fp16_slot[li][4..8]). */
typedef struct {
    const float *tap_q, *tap_k, *tap_v;
    const float *norm_q, *norm_k;
} ndo_front_w;

/* Give a session the front state: taps >= 1 histories (zeroed) and the
 * rotary table for rope_theta. 0 ok, negative on bad arguments / no memory. */
int  ndo_session_front(ndo_session *s, uint32_t taps, float rope_theta);
/* The front for layer li at s->pos, in place on q [nh*qk_hd], k [nkv*qk_hd],
 * v [nkv*v_hd] (raw projections in, store-ready rows out). */
void ndo_front(ndo_session *s, uint32_t li, const ndo_front_w *w, float *q, float *k, float *v);

/* ---- CQ projections (engine/src/nd_quant.c, engine/include/nd_quant.h) ----
 *
 * A CQ tensor [out][in] stores per group of `group` weights a `bits`-wide
 * codebook index per weight (an LSB-first bitstream per row, rows of
 * in_pad*bits/8 bytes, in_pad = in rounded up to group) and one fp16 norm
 * per (row, group), the norms [out][in_pad/group] following the packed rows
 * in the same blob. w_group = (cb[idx] * norm) @ H with H the orthonormal
 * Walsh-Hadamard matrix, so a matvec transforms the activation instead:
 * xh = H x per group, y[o] = sum_g norm[o][g] * sum_i cb[idx[o][i]] * xh[i].
 * cb is the archive's codebook slice for the width (2^bits entries, already
 * scaled by 1/sqrt(group)). */
uint32_t ndo_cq_in_pad(uint32_t in, uint32_t group);
/* In-place unnormalised fast Walsh-Hadamard transform, n a power of two
 * (nd_fwht, nd_quant.c:36-65). */
void ndo_fwht(float *x, uint32_t n);
/* xh[in_pad] = x zero-padded, then per group H scaled by 1/sqrt(group)
 * (nd_cq_prepare, nd_quant.c:354-387; fwht_rows / fw_scale :99-116, :303-352). */
void ndo_cq_prepare(uint32_t in, uint32_t group, const float *x, float *xh);
/* y[out] = W . x for a prepared xh: the generic row walker and its group dot
 * (gemv_rows_generic :616-632, dot_group :389-462). */
void ndo_cq_gemv(uint32_t out, uint32_t in, uint32_t group, uint32_t bits, const void *blob,
                 const float *cb, const float *xh, float *y);
/* The 2-bit pair table: lut[p*16 + i0 + 4*i1] = cb[i0]*xh[2p] + cb[i1]*xh[2p+1]
 * (nd_cq_lut_build / lutb_rows, :75-97, :800-807). */
void ndo_cq_lut_build(const float *cb2, const float *xh, uint32_t in_pad, float *lut);
/* y[out] = W . x for a 2-bit tensor through the pair table (nd_cq_gemv_lut2 /
 * nd_lut2_rows_c, :734-773, :809-839). */
void ndo_cq_gemv_lut2(uint32_t out, uint32_t in, uint32_t group, const void *blob,
                      const float *lut, float *y);

/* ---- the whole attention block (attention(), nd_model.c:2382-2502) ----
 * One layer's five 2-bit CQ projections (blob[0..4]: q, k, v, gate, out_proj,
 * the archive's payloads), the 2-bit codebook slice, d_model and the group. */
typedef struct {
    const void *blob[5];
    const float *cb2;
    uint32_t d_model, group;
} ndo_block_w;

/* attention(m, li, xin, out) at s->pos: prepare + pair table + q/k/v/gate
 * (nd_model.c:2397-2411), the front (:2413-2424), the store and attn_heads
 * with the gate (:2426-2483), prepare + out_proj (:2495-2501).
 * xin [d_model] -> out [d_model]. Needs ndo_session_front. */
int ndo_attention_block(ndo_session *s, uint32_t li, const ndo_front_w *fw, const ndo_block_w *bw,
                        const float *xin, float *out);

/* ---- CPU baseline: batched fp16 decode, threaded over sequences ----
 *
 * Independent sequences b in [0, nseq): K/V in a contiguous per-sequence slot
 * array k[b] = kbase + koff[b] (elements), window = len[b] slots, n_sink 0,
 * pos = len[b]-1. The new token's K/V (k_new/v_new fp32) is stored at slot
 * len[b]-1 first, as the engine does, then attended. nthreads workers take whole
 * sequences (the nd_parallel_rows seam, nd_quant.h:213-230). */
typedef struct {
    uint32_t nseq, nh, nkv, qk_hd, v_hd;
    const uint32_t *len;
    const uint64_t *koff, *voff;
    uint16_t *kbase, *vbase;
    const float *q, *k_new, *v_new, *gate;   /* per sequence: nh*qk_hd, nkv*qk_hd, nkv*v_hd, nh*v_hd */
    float *out;                              /* nseq*nh*v_hd */
} ndo_batch_f16;

int ndo_decode_batch_f16(const ndo_batch_f16 *b, int nthreads);

/* Causal prefill restated as the engine runs it: one token at a time through
 * ndo_attention (esp32/main/main.c:312-315). q/k/v/gate/out are [n][...]. */
void ndo_prefill_tokens(ndo_session *s, uint32_t li, uint32_t n, const float *q,
                        const float *k, const float *v, const float *gate, float *out);

#ifdef __cplusplus
}
#endif
#endif
