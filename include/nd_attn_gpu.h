/* nd_attn_gpu.h - the engine-side C shim: one Needle session's attention and
 * KV-cache state on the GPU, driven with the engine's own host arrays.
 *
 * Each function mirrors one reference entry point for the attention path,
 * with the same argument meaning and error behaviour (0 / negative codes,
 * NULL on failure for the prefix handle):
 *
 *   nd_gpu_reset          nd_model_reset          engine/src/nd_model.c:1557-1581
 *   nd_gpu_set_sink       nd_model_set_sink       :1314-1321
 *   nd_gpu_snapshot       nd_model_snapshot       :1395-1434
 *   nd_gpu_rewind         nd_model_rewind         :1436-1460
 *   nd_gpu_prefix_save    nd_model_prefix_save    :1531-1541
 *   nd_gpu_prefix_restore nd_model_prefix_restore :1543-1553
 *   nd_gpu_prefix_free    nd_model_prefix_free    :1555
 *   nd_gpu_attention      the KV store + attn_heads dispatch of attention()
 *                         :2426-2483 (m->q, m->kbuf, m->vbuf, m->gate -> m->attn)
 *   nd_gpu_step_end       pos++ at the end of nd_model_step_hidden :3094
 *   nd_gpu_front_init     the tap histories (:1178-1180) and rotary
 *                         frequencies (:1233-1236) that nd_model_open sets up
 *   nd_gpu_front_weights  one layer's staged tap weights and q/k norm scales
 *                         (fp16_slot[li][4..8])
 *   nd_gpu_attention_raw  attention() after the projections :2413-2483: tap
 *                         convolution, head norm + RoPE, KV store, attn_heads
 *                         and the gate, from the raw m->q, m->kbuf, m->vbuf
 *   nd_gpu_block_weights  one layer's q/k/v/gate/out_proj CQ tensors
 *   nd_gpu_attention_block  the whole attention(m, li, xin, out) :2382-2502:
 *                         CQ projections, the front (if initialised), store,
 *                         attention, gate, out_proj
 *
 * The KV part of the session state lives here, and with the front
 * initialised the qkv tap histories too; the rest of the prefix state
 * (engram, confidence pool) stays with the engine.
 */
#ifndef ND_ATTN_GPU_H
#define ND_ATTN_GPU_H

#include <stdint.h>

#include "nda.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nd_gpu_model nd_gpu_model;
typedef struct nd_gpu_prefix nd_gpu_prefix;

/* Geometry as the engine's nd_model fields; kv_dtype NDA_KV_INT8 is the
 * engine's own cache format. max_prefixes bounds live prefix caches. */
nd_gpu_model *nd_gpu_open(uint32_t n_layers, uint32_t n_heads, uint32_t n_kv_heads,
                          uint32_t qk_head_dim, uint32_t v_head_dim, uint32_t window,
                          uint32_t kv_dtype, uint32_t max_prefixes);
void nd_gpu_close(nd_gpu_model *m);

void nd_gpu_reset(nd_gpu_model *m);
void nd_gpu_set_sink(nd_gpu_model *m, uint32_t n);
int  nd_gpu_snapshot(nd_gpu_model *m);
void nd_gpu_rewind(nd_gpu_model *m);
nd_gpu_prefix *nd_gpu_prefix_save(nd_gpu_model *m);
int  nd_gpu_prefix_restore(nd_gpu_model *m, const nd_gpu_prefix *p);
void nd_gpu_prefix_free(nd_gpu_prefix *p);

/* Host arrays, the engine's layout: q [nh*qk_hd], k [nkv*qk_hd],
 * v [nkv*v_hd], gate [nh*v_hd] (NULL: no gate), out [nh*v_hd]. */
int  nd_gpu_attention(nd_gpu_model *m, uint32_t li, const float *q, const float *k,
                      const float *v, const float *gate, float *out);
/* The attention front: after nd_gpu_front_init (taps 1..8, max_pos 0 for
 * 65536) and nd_gpu_front_weights for every layer, nd_gpu_attention_raw takes
 * the RAW projections (before tap_projection / zcrms_heads) in the same
 * layout as nd_gpu_attention. Snapshot, rewind, prefix save / restore and
 * reset carry the tap histories as the engine does. */
int  nd_gpu_front_init(nd_gpu_model *m, uint32_t taps, float rope_theta, uint32_t max_pos);
int  nd_gpu_front_weights(nd_gpu_model *m, uint32_t li, const float *tap_q, const float *tap_k,
                          const float *tap_v, const float *norm_q, const float *norm_k);
int  nd_gpu_attention_raw(nd_gpu_model *m, uint32_t li, const float *q, const float *k,
                          const float *v, const float *gate, float *out);
/* The whole block: register each layer's CQ tensors (nda_cq_create from the
 * archive's q_proj, k_proj, v_proj, gate_proj, out_proj; borrowed), then
 * nd_gpu_attention_block takes the layer's normalised input xin [d_model]
 * and writes attention()'s output out [d_model] (host arrays). */
int  nd_gpu_block_weights(nd_gpu_model *m, uint32_t li, const nda_cq *q, const nda_cq *k,
                          const nda_cq *v, const nda_cq *gate, const nda_cq *out_proj);
int  nd_gpu_attention_block(nd_gpu_model *m, uint32_t li, const float *xin, uint32_t d_model,
                            float *out);
void nd_gpu_step_end(nd_gpu_model *m);

uint32_t nd_gpu_pos(const nd_gpu_model *m);
uint32_t nd_gpu_n_sink(const nd_gpu_model *m);
/* The context underneath, for inspection (nda_kv_read). Sequence 0. */
nda_ctx *nd_gpu_ctx(nd_gpu_model *m);

#ifdef __cplusplus
}
#endif
#endif
