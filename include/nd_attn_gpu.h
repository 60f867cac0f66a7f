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
 *
 * Only the KV part of the session state lives here; the non-KV prefix state
 * (conv taps, engram, confidence pool) stays with the engine.
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
void nd_gpu_step_end(nd_gpu_model *m);

uint32_t nd_gpu_pos(const nd_gpu_model *m);
uint32_t nd_gpu_n_sink(const nd_gpu_model *m);
/* The context underneath, for inspection (nda_kv_read). Sequence 0. */
nda_ctx *nd_gpu_ctx(nd_gpu_model *m);

#ifdef __cplusplus
}
#endif
#endif
