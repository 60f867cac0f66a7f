/* nda.h - C ABI of libndattn: the Needle engine's attention / KV-cache hot
 * path on MI355X (gfx950).
 *
 * The engine (iammrduncan/esp32-needle-3) keeps one session's KV cache as a
 * per-layer ring of `window` int8 slots with an fp32 scale per (slot, kv-head)
 * and attends with attn_heads behind the nd_parallel_rows row seam. This
 * library holds the KV of many independent sequences in paged HBM and runs
 * the same operations batched across them. Every entry point below names the
 * reference interface it replaces.
 *
 * Conventions (engine/include/nd_model.h:191-236, nd_model.c:760-767):
 *   - every function returns 0 on success or a negative NDA_ERR_* code; no C++
 *     exception or HIP error crosses the ABI; nda_last_error() explains the
 *     last failure on a context;
 *   - q, k, v, gate and out are DEVICE pointers (fp32) unless stated;
 *     seq_ids and n_tokens are HOST arrays (NULL seq_ids = sequences 0..nseq-1);
 *   - stream is a hipStream_t passed as void* (NULL = the default stream);
 *   - a context is used by one host thread at a time; calls on it are serial.
 *     Kernels launched by one call write disjoint (sequence, head) outputs;
 *   - calls on one context are ordered as if they ran on one stream (the
 *     engine's single-threaded contract, engine/include/nd_quant.h:221-228):
 *     a call on a stream other than the previous call's first makes its
 *     stream wait for the work queued on the previous one, so that stream
 *     must still exist then (nda_sync on it releases that). The inspection
 *     calls (nda_kv_read / nda_kv_write) run on the null stream the same way.
 *     Contexts do not order each other.
 */
#ifndef NDA_H
#define NDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NDA_OK               0
#define NDA_ERR_ARG         -1   /* bad argument or geometry */
#define NDA_ERR_NOMEM       -2   /* device memory or page pool exhausted */
#define NDA_ERR_HIP         -3   /* a HIP runtime call failed */
#define NDA_ERR_RANGE       -4   /* position / length outside what the window holds */
#define NDA_ERR_STATE       -5   /* call not valid in the sequence's current state */
#define NDA_ERR_UNSUPPORTED -6   /* a shape the engine does not define, or a CQ tensor form
                                    (bits, group, width) the call does not take */
#define NDA_ERR_NODEV       -7   /* no usable gfx950 device */

/* KV element types. INT8: symmetric int8 codes + fp32 scale per (slot,
 * kv-head), the engine's own format (nd_model.h:17-20, :134-137). F16: IEEE
 * half, scale 1 (the fp16 variant of the same path). */
#define NDA_KV_INT8 0
#define NDA_KV_F16  1

typedef struct nda_ctx nda_ctx;

/* Geometry and capacities. Mirrors the engine's model shape fields
 * (nd_model.h:89-90: n_layers, n_heads, n_kv_heads, qk_head_dim, v_head_dim,
 * window) plus the batched-serving capacities the engine does not have. */
typedef struct {
    uint32_t n_layers;
    uint32_t n_heads;        /* query heads */
    uint32_t n_kv_heads;     /* n_heads % n_kv_heads == 0, at most 8 query heads per
                                kv-head (ND_KV_REP_CAP, nd_model.h:245) */
    uint32_t qk_head_dim;    /* 4..64, a multiple of 4 (ND_KV_HD_CAP, nd_model.h:244; the
                                engine's staging converts whole 4-byte words, nd_model.c:79-94) */
    uint32_t v_head_dim;     /* 4..64, a multiple of 4 */
    uint32_t window;         /* KV slots per sequence per layer (sinks + ring) */
    uint32_t page_size;      /* positions per page: 16, 32 or 64 (0 = 16) */
    uint32_t kv_dtype;       /* NDA_KV_INT8 | NDA_KV_F16 */
    uint32_t max_seqs;       /* sequence slots */
    uint32_t max_prefixes;   /* shared prefix segments (0 = 16) */
    uint64_t max_pages;      /* page pool size per layer (0 = enough for every
                                sequence's full window plus the prefixes) */
    uint32_t split_chunk;    /* positions per split-KV work item (0 = auto) */
    uint32_t flags;          /* NDA_FLAG_* */
} nda_config;

/* Prefill through the per-row VALU decode kernel instead of the MFMA
 * kernel (same results within rounding; for comparison and tiny chunks). */
#define NDA_FLAG_PREFILL_VALU 1u
/* Decode GQA groups (4 or more query heads per kv-head) through the VALU
 * decode kernel instead of the MFMA one (same results within rounding; for
 * comparison). */
#define NDA_FLAG_DECODE_VALU 2u

/* ---- lifecycle ---- */

/* Allocates the paged KV pool and tables on the current HIP device.
 * Replaces the KV part of nd_model_open (nd_model.c:1142-1144, :1195-1198). */
int  nda_create(const nda_config *cfg, nda_ctx **out);
void nda_destroy(nda_ctx *ctx);
const char *nda_last_error(const nda_ctx *ctx);
/* Bytes of device memory the context holds (pool + tables + scratch). */
uint64_t nda_device_bytes(const nda_ctx *ctx);

/* ---- per-sequence session state (host-side mirror, uploaded lazily) ---- */

/* nd_model_reset (nd_model.c:1557-1581), KV part: pos = 0, n_sink = 0, no
 * snapshot, detached from any shared prefix, pages returned to the pool. */
int nda_seq_reset(nda_ctx *ctx, uint32_t seq);
/* nd_model_set_sink (nd_model.c:1314-1321): pin the first n positions,
 * clamped to window - 64. */
int nda_seq_set_sink(nda_ctx *ctx, uint32_t seq, uint32_t n);
int nda_seq_state(const nda_ctx *ctx, uint32_t seq, uint32_t *pos, uint32_t *n_sink,
                  int32_t *prefix_id);
/* Sets pos directly (a sequence whose KV was written through nda_kv_write). */
int nda_seq_set_pos(nda_ctx *ctx, uint32_t seq, uint32_t pos);
/* Back the slots of positions [pos, pos + n) with pages now, so that later
 * appends allocate nothing. No counterpart in the engine (its cache is one
 * flat allocation). */
int nda_seq_reserve(nda_ctx *ctx, uint32_t seq, uint32_t n);
/* End of a token for these sequences: pos += n. The engine does pos++ at the
 * end of nd_model_step_hidden (nd_model.c:3094), after every layer. The
 * device copy is incremented in stream order (no upload). */
int nda_advance(nda_ctx *ctx, uint32_t nseq, const uint32_t *seq_ids, uint32_t n, void *stream);

/* ---- shared prefix (schema) segments ---- */

/* nd_model_snapshot + nd_model_prefix_save (nd_model.c:1395-1434, :1531-1541):
 * pins the sequence's current positions as sinks and copies its live KV into
 * a read-only segment any number of sequences can then share. */
int nda_prefix_build(nda_ctx *ctx, uint32_t seq, int32_t *prefix_id, void *stream);
/* nd_model_prefix_restore (nd_model.c:1543-1553): the sequence resumes at the
 * prefix's position with its sinks read from the shared segment - no copy of
 * the pinned positions. Positions past the sink clamp are copied into the
 * sequence's own ring, as the engine restores them. */
int nda_seq_attach(nda_ctx *ctx, uint32_t seq, int32_t prefix_id, void *stream);
/* nd_model_rewind (nd_model.c:1436-1460), KV part: back to the attached
 * prefix's position (or reset when none). */
int nda_seq_rewind(nda_ctx *ctx, uint32_t seq);
/* nd_model_prefix_free. Fails with NDA_ERR_STATE while sequences use it. */
int nda_prefix_free(nda_ctx *ctx, int32_t prefix_id);

/* ---- the hot path ---- */

/* Store each sequence's K/V for its current position into layer `layer`:
 * k [nseq][n_kv_heads][qk_head_dim], v [nseq][n_kv_heads][v_head_dim] fp32.
 * INT8 quantises per kv-head exactly as the engine does (absmax/127 scale,
 * correctly rounded divide, clamp, round-half-even; nd_model.c:2426-2449 and
 * kv_store_int8 :1819-1866); F16 rounds to nearest even. Allocates a page
 * when the slot's page is not backed yet. */
int nda_kv_append(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
                  const float *k, const float *v, void *stream);

/* Single-token attention at each sequence's current position over its sinks
 * and recent ring, GQA, online softmax, gated emit:
 * q [nseq][n_heads][qk_head_dim], gate [nseq][n_heads][v_head_dim] or NULL
 * (no output gate), out [nseq][n_heads][v_head_dim] fp32.
 * Replaces nd_parallel_rows(attn_heads, &actx, nh) in attention()
 * (nd_model.c:2451-2483, attn_heads :2105-2359). */
int nda_decode(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
               const float *q, const float *gate, float *out, void *stream);

/* Bytes of the per-GPU scratch array nda_decode_noalloc works in. */
#define NDA_NOALLOC_SCRATCH_BYTES (16u << 20)

/* nda_decode that allocates nothing: no counterpart in the reference. For
 * callers that must not allocate device memory (tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments as nda_decode, and the
 * same results within fp32 rounding: the same kernels, except that it never
 * takes the shared-prefix decode pass (a batch on one shared prefix is then
 * attended row by row) or the longest-first row order of the GQA decode,
 * whose work buffers the context grows. The sequence ids and the split-KV
 * partials (long rows cut into
 * chunks merged by log-sum-exp) live in one static device array of
 * NDA_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, instead of
 * context buffers grown by hipMalloc. A call whose ids (4 bytes each, after
 * 256-byte alignment) plus partials (rows * n_heads * chunks * (v_head_dim +
 * 2) floats) exceed it returns NDA_ERR_RANGE and changes nothing. Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other contexts, other host threads) race. Records no profiling
 * events. */
int nda_decode_noalloc(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
                       const float *q, const float *gate, float *out, void *stream);

/* nda_kv_append + nda_decode, in the order attention() runs them (store
 * first; the current token is attended). Small batches, and batches on one
 * shared prefix that take the prefix pass, store inside the decode launch;
 * other large ones run the two kernels; the results are the same. */
int nda_step(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
             const float *q, const float *k, const float *v, const float *gate,
             float *out, void *stream);

/* Causal prefill of n_tokens[b] new tokens per sequence at positions
 * [pos, pos + n): appends their K/V, then token t attends exactly what a
 * decode at position pos + t would (the engine prefills by repeated
 * nd_model_step_hidden: esp32/main/main.c:233-234, :312-315). Inputs are
 * packed token-major per sequence, sequence b's rows starting at
 * sum(n_tokens[0..b)): q [T][n_heads][qk_head_dim], k [T][n_kv_heads][qk_head_dim],
 * v [T][n_kv_heads][v_head_dim], gate/out [T][n_heads][v_head_dim].
 * Requires pos + n <= window (no ring wrap inside the chunk): NDA_ERR_RANGE
 * otherwise; q and out 16-byte aligned (NDA_ERR_ARG). Does not advance pos. */
int nda_prefill(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
                const uint32_t *n_tokens, const float *q, const float *k, const float *v,
                const float *gate, float *out, void *stream);

int nda_sync(nda_ctx *ctx, void *stream);

/* ---- attention front (engine/src/nd_model.c:2413-2424) ----
 * What attention() does to the raw q/k/v projections before the store:
 * tap_projection for q, k and v (:2361-2379, tap_rows :1748-1802), a causal
 * depthwise convolution of every column over its last `taps` raw values,
 * then zcrms_heads for q and k (:324-360), a per-head RMS norm with a
 * (1 + s) scale shared by all heads, fused with half-split RoPE at the
 * token's position. Results are bit-identical to the engine's host build.
 * The raw projections of the last `taps` positions of each sequence and
 * layer (the engine's q_hist/k_hist/v_hist, nd_model.h:167) live on the
 * device and follow the sequence through nda_seq_reset (zeroed),
 * nda_prefix_build / nda_seq_attach (saved with the prefix and restored,
 * as nd_model_prefix_save / restore do, :1519-1521) and nda_seq_rewind. */
typedef struct {
    uint32_t taps;         /* the archive's qkv_conv_taps, 1..8 */
    float    rope_theta;   /* the archive's rope_theta */
    uint32_t max_pos;      /* the rotary table covers positions [0, max_pos); 0: 65536 */
} nda_front_config;

/* Allocates the tap histories and the rotary table (cos/sin of
 * pos * theta^(-2i/qk_head_dim), as nd_model_open :1233-1236 and
 * nd_model_step_hidden :2949-2954 compute them). Once per context. Every
 * shape the context accepts has a front (qk/v 64/64 and 48/64 on kernels
 * specialised for them, the others with their dims read at run time). */
int nda_front_init(nda_ctx *ctx, const nda_front_config *fc);
/* One layer's weights from HOST arrays, the engine's staged fp32 slots
 * (fp16_slot[li][4..8]): tap_q [taps][n_heads*qk_head_dim],
 * tap_k [taps][n_kv_heads*qk_head_dim], tap_v [taps][n_kv_heads*v_head_dim],
 * norm_q / norm_k [qk_head_dim]. */
int nda_front_weights(nda_ctx *ctx, uint32_t layer, const float *tap_q, const float *tap_k,
                      const float *tap_v, const float *norm_q, const float *norm_k);
/* The front for n_tokens[b] tokens of each listed sequence at positions
 * pos, pos+1, ... (n_tokens NULL: one token each), packed token-major as
 * nda_prefill's inputs: raw q/k/v in, q_out/k_out/v_out (same shapes, device)
 * out, ready for nda_step / nda_prefill. Updates the tap histories; does not
 * advance pos. Each sequence at most once per call. */
int nda_front(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
              const uint32_t *n_tokens, const float *q, const float *k, const float *v,
              float *q_out, float *k_out, float *v_out, void *stream);
/* attention() from the raw projections on: the front, the KV store of this
 * position and the decode, for one token of each listed sequence. q/k/v raw
 * [nseq][...], gate/out as nda_decode. Does not advance pos. */
int nda_attention(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
                  const float *q, const float *k, const float *v, const float *gate,
                  float *out, void *stream);
/* Copies one sequence's tap histories (snap 0: live, 1: the snapshot that
 * nda_seq_rewind restores) to a HOST buffer
 * [n_layers][taps][n_heads*qk_head_dim + n_kv_heads*(qk_head_dim + v_head_dim)]. */
int nda_front_hist(nda_ctx *ctx, uint32_t seq, int snap, float *dst, void *stream);

/* ---- CQ projections (engine/src/nd_quant.c, engine/include/nd_quant.h) ----
 * The engine's codebook-quantised matvecs for a batch of rows. A CQ tensor
 * [out][in] is the archive's blob: per row an LSB-first bitstream of `bits`
 * -wide codebook indices over in_pad = in rounded up to `group`, then the
 * fp16 norms [out][in_pad/group]; the weights are
 * w_group = (codebook[idx] * norm) @ H, H the orthonormal Walsh-Hadamard
 * matrix of size group. As in the engine, the activation is transformed
 * (nda_cq_prepare, nd_cq_prepare) and the transformed rows are multiplied
 * against the codes (nda_cq_gemm: nd_cq_gemv_prepared / nd_cq_gemv_lut2,
 * for every row of the batch). q/k/v/gate and out_proj of attention()
 * (nd_model.c:2402-2411, :2495-2501) are such tensors at 2 bits. */
typedef struct nda_cq nda_cq;

/* Copies one tensor to the device. blob: host, the tensor payload (packed
 * rows then norms); codebook: host, the 2^bits entries for this width
 * (nd_cact_codebook). group a power of two in 16..4096, bits 2..4. A 2-bit
 * tensor with group >= 32 also gets the split path's decode data, built on
 * the device before the call returns (a kernel on the null stream, then a
 * wait on it): its codes re-ordered into per-lane words (the size of the
 * packed codes), and per (row, group) the four weights codebook[c] * norm
 * as fp16 pairs (16 bytes), with one exponent per row. */
int nda_cq_create(uint32_t out, uint32_t in, uint32_t group, uint32_t bits, const void *blob,
                  const float *codebook, nda_cq **t);
int nda_cq_destroy(nda_cq *t);
/* in_pad of the tensor (the prepared row length). */
uint32_t nda_cq_in_pad(const nda_cq *t);
/* xh[rows][in_pad] = per-group H of x[rows][in] zero-padded (device
 * pointers, 16-byte aligned). Bit-identical to nd_cq_prepare. Reusable by
 * every tensor with the same (in, group). */
int nda_cq_prepare(const nda_cq *t, uint32_t rows, const float *x, float *xh, void *stream);
/* y[rows][out] = W . x for each row, from its prepared xh (device pointers). */
int nda_cq_gemm(const nda_cq *t, uint32_t rows, const float *xh, float *y, void *stream);
/* The same for n <= 8 tensors that share the prepared activation (same in,
 * group and bits: q/k/v/gate of one layer), in one launch: y_i = W_i . x
 * into ys[i][rows][out_i]. */
int nda_cq_gemm_many(const nda_cq *const *ts, uint32_t n, uint32_t rows, const float *xh, float *const *ys,
                     void *stream);
/* The same matvecs (nd_cq_prepare + nd_cq_gemv_lut2, for every row) on fp16
 * MFMA with split operands, for 2-bit tensors with group >= 32 (otherwise
 * NDA_ERR_UNSUPPORTED). The prepared form xs (device, 16-byte aligned,
 * nda_cq_split_bytes) holds per row the engine's prepared values times a
 * power of two 2^e as an fp16 pair hi + lo: plane hi [rows][in_pad], plane
 * lo [rows][in_pad], then e [rows] (int32). The weights codebook[c] * norm
 * are split the same way, per (row, group), when the tensor is created; the
 * fourth product (lo x lo, 2^-22 relative) is dropped, so the result is
 * within a few 2^-22 of sum |w x| of the engine's. The attention block calls
 * take this path above 64 rows when all five tensors allow it. */
size_t nda_cq_split_bytes(const nda_cq *t, uint32_t rows);
int nda_cq_prepare_split(const nda_cq *t, uint32_t rows, const float *x, void *xs, void *stream);
int nda_cq_gemm_split(const nda_cq *t, uint32_t rows, const void *xs, float *y, void *stream);
int nda_cq_gemm_split_many(const nda_cq *const *ts, uint32_t n, uint32_t rows, const void *xs,
                           float *const *ys, void *stream);
/* The engine's own 2-bit matvec, bit for bit: nd_cq_lut_build +
 * nd_cq_gemv_lut2 (engine/src/nd_quant.c:667-677, :809-821; the table rows
 * lutb_rows :75-94, the row walk nd_lut2_rows_c :722-764) for each row of xh (nda_cq_prepare's form,
 * device, 16-byte aligned): y_i = W_i . x into ys[i][rows][out_i] for
 * n <= 8 tensors sharing in and group, 2-bit, in_pad <= 2048, rows <=
 * 65535 (otherwise NDA_ERR_UNSUPPORTED). Each output is a serial sum, so
 * this is the path for a few rows (one token per sequence); the attention
 * block calls take it for at most 64 rows, where the stored int8 codes then
 * equal the engine's exactly. */
int nda_cq_gemv_lut2(const nda_cq *const *ts, uint32_t n, uint32_t rows, const float *xh, float *const *ys,
                     void *stream);

/* ---- the whole attention block (attention(), engine/src/nd_model.c:2382-2502) ----
 * Register one layer's five CQ tensors (borrowed: they must outlive the
 * context's use of them): q [nh*qk][d_model], k [nkv*qk][d_model],
 * v [nkv*v][d_model], gate [nh*v][d_model], out_proj [d_model][nh*v], all
 * with one group and width. */
int nda_block_weights(nda_ctx *ctx, uint32_t layer, const nda_cq *q, const nda_cq *k, const nda_cq *v,
                      const nda_cq *gate, const nda_cq *out_proj);
/* attention() for one token of each listed sequence: x [nseq][d_model] (the
 * layer's normalised input) -> q/k/v/gate projections -> the front (when
 * initialised; raw projections otherwise go straight to the store) -> KV
 * store + decode with the gate -> out_proj -> out [nseq][d_model]. Device
 * pointers, 16-byte aligned. Does not advance pos. */
int nda_attention_block(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
                        const float *x, float *out, void *stream);
/* The same block for a chunk of n_tokens[b] tokens of each listed sequence
 * at positions pos, pos+1, ..., all tokens of the layer at once: what
 * n_tokens[b] successive attention() calls of this layer compute (the engine
 * prefills one token at a time: esp32/main/main.c:233-234, :312-315; taps
 * and the KV store depend only on earlier tokens, so a layer can take the
 * chunk in one pass). x / out [T][d_model], packed token-major per sequence
 * as nda_prefill's inputs, device, 16-byte aligned. The projections run
 * over all T rows, the front over each sequence's chunk, then nda_prefill
 * (store + causal attention with the gate) and out_proj. Requires
 * pos + n <= window (NDA_ERR_RANGE); rejected chunks, and a full page pool,
 * change nothing. Does not advance pos. */
int nda_prefill_block(nda_ctx *ctx, uint32_t layer, uint32_t nseq, const uint32_t *seq_ids,
                      const uint32_t *n_tokens, const float *x, float *out, void *stream);

/* ---- stream-ordered timing ---- */
int nda_event_create(void **ev);
int nda_event_destroy(void *ev);
int nda_event_record(void *ev, void *stream);
/* Milliseconds between two recorded events (waits for the second). */
int nda_event_elapsed(void *start, void *stop, float *ms);

/* ---- inspection (tests, tools) ---- */

/* Copies the stored K/V of `count` consecutive positions starting at
 * position p0 of one sequence and layer to HOST buffers:
 * k [count][n_kv_heads][qk_head_dim] and v [...][v_head_dim] in the KV
 * element type (int8 or fp16 bits), k_scale/v_scale [count][n_kv_heads]
 * (NULL allowed; all 1.0 for F16). Positions must be currently visible. */
int nda_kv_read(nda_ctx *ctx, uint32_t layer, uint32_t seq, uint32_t p0, uint32_t count,
                void *k, void *v, float *k_scale, float *v_scale);
/* The reverse: write stored-format K/V for positions [p0, p0+count) (pages are
 * allocated as needed). Used to load an existing cache. */
int nda_kv_write(nda_ctx *ctx, uint32_t layer, uint32_t seq, uint32_t p0, uint32_t count,
                 const void *k, const void *v, const float *k_scale, const float *v_scale);

/* Fills the stored K/V of positions [0, pos) of every listed sequence, every
 * layer, with N(0,1) values from a counter-based generator keyed by (seed,
 * layer, sequence, position, head, element) - independent of page placement.
 * INT8: codes round(32 x) clamped to +-127, scales 1/32. Synthetic benchmark
 * data. */
int nda_kv_fill_normal(nda_ctx *ctx, uint32_t nseq, const uint32_t *seq_ids, uint64_t seed,
                       void *stream);

/* ---- device memory ---- */

/* The device allocator every context, CQ tensor and nda_dev_alloc block is
 * taken from: alloc returns `bytes` of device memory (16-byte aligned) or
 * NULL, free releases a block alloc returned. Replaces the engine's platform
 * allocation seams ND_ALLOC / ND_FREE (nd_model.h:35-68), which pick where
 * its KV cache and scratch live; here they are set at run time for the
 * process. NULL, NULL restores hipMalloc / hipFree. Blocks are freed through
 * the free function current at that time, so switch only between
 * allocators that can free each other's blocks (for example wrappers of one
 * underlying allocator). A call that cannot get the memory it needs returns
 * NDA_ERR_NOMEM and changes no session state. */
typedef void *(*nda_alloc_fn)(size_t bytes, void *user);
typedef void (*nda_free_fn)(void *ptr, void *user);
int nda_set_allocator(nda_alloc_fn alloc, nda_free_fn free_fn, void *user);

/* Device plumbing for hosts without their own allocator (through the
 * allocator above). */
int nda_dev_alloc(void **ptr, size_t bytes);
int nda_dev_free(void *ptr);
int nda_h2d(void *dst, const void *src, size_t bytes);
int nda_d2h(void *dst, const void *src, size_t bytes);
int nda_memset(void *dst, int value, size_t bytes);
/* Page-locked host memory, and stream-ordered copies to / from it (from
 * pageable memory they complete before returning). */
int nda_host_alloc(void **ptr, size_t bytes);
int nda_host_free(void *ptr);
int nda_h2d_async(void *dst, const void *src, size_t bytes, void *stream);
int nda_d2h_async(void *dst, const void *src, size_t bytes, void *stream);
/* Device-to-device copy on a stream (also the known-size copy used to
 * calibrate memory-traffic counters). */
int nda_d2d(void *dst, const void *src, size_t bytes, void *stream);
/* dst[i] = N(0,1) * scale as fp32 (dtype 0) or fp16 (dtype 1), i < n;
 * counter-based (seed, i). */
int nda_fill_normal(void *dst, uint64_t n, int dtype, uint64_t seed, float scale, void *stream);
int nda_stream_create(void **stream);
int nda_stream_destroy(void *stream);
int nda_device_sync(void);
/* Device name and compute-unit count of the current device. */
int nda_device_info(char *name, size_t name_len, int *cu_count);

/* ---- kernel timing (the engine's ND_PROFILE phases, nd_model.h:238-269) ----
 * When enabled, every launch is bracketed by HIP events on its own stream and
 * the elapsed device time is accumulated per kernel kind. */
#define NDA_K_APPEND  0   /* ND_P_KVST */
#define NDA_K_DECODE  1   /* ND_P_ATTN */
#define NDA_K_COMBINE 2   /* split-KV merge */
#define NDA_K_PREFILL 3
#define NDA_K_FRONT   4   /* ND_P_TAPS + ND_P_HNORM (+ the store in nda_attention) */
#define NDA_K_PROJ    5   /* ND_P_PREP + ND_P_PROJ: CQ prepare and matvec launches of nda_attention_block */
#define NDA_K_COUNT   6
int nda_prof_enable(nda_ctx *ctx, int on);
/* Synchronises outstanding timed launches, then returns per kind the summed
 * milliseconds and launch counts; resets when reset != 0. */
int nda_prof_read(nda_ctx *ctx, double ms[NDA_K_COUNT], uint64_t launches[NDA_K_COUNT], int reset);

#ifdef __cplusplus
}
#endif
#endif /* NDA_H */
