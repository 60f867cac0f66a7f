/* nda_internal.h - shared definitions between the C-ABI layer (nda_api_*.hip)
 * and the gfx950 kernels (nda_kernels.hip, nda_prefill.hip, nda_front.hip,
 * nda_cq.hip). Not installed. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nda {

/* Per-sequence state as the kernels see it. pos is the position being
 * stored/attended (the engine's m->pos), n_sink the pinned count, prefix the
 * shared segment id or -1. */
struct SeqDev {
    int32_t pos;
    int32_t n_sink;
    int32_t prefix;
    int32_t pad;
};

/* Page geometry of one layer pool. A page holds page_size consecutive slots
 * of one sequence (or prefix) for every kv-head:
 *   page + g*head_bytes:  K codes   [page_size][dk]
 *                         V codes   [page_size][dv]
 *                         K scales  [page_size] fp32   (int8 only)
 *                         V scales  [page_size] fp32   (int8 only)      */
struct PageGeom {
    uint32_t log2_page;     /* page_size = 1 << log2_page */
    uint32_t pages_per_seq; /* page-table row length = ceil(window / page_size) */
    uint64_t head_bytes;
    uint64_t page_bytes;
    uint64_t layer_bytes;   /* page_bytes * max_pages */
    uint32_t window;
    uint32_t nkv;
    uint32_t dk, dv;        /* qk_head_dim, v_head_dim */
};

/* One launch of the decode / causal kernel. A "row" is one query token of
 * one sequence: batch index b = row_seq_idx, visible position = pos + row_t. */
struct AttnArgs {
    const float *q;          /* [rows][nh][dk] */
    const float *gate;       /* [rows][nh][dv] or null */
    float *out;              /* [rows][nh][dv] */
    const uint8_t *pool;     /* this layer's pool base */
    const int32_t *page_table;
    const int32_t *prefix_pages;
    const SeqDev *seqs;
    const uint32_t *row_seq; /* [rows] sequence id per row, or null: row -> seq_ids/identity */
    const uint32_t *row_t;   /* [rows] offset from pos, or null: 0 */
    float *part;             /* split partials [rows][nh][max_chunks][dv + 2] */
    PageGeom pg;
    uint32_t rows;
    uint32_t nh;
    uint32_t chunk;          /* positions per work item */
    uint32_t max_chunks;
    uint32_t chunk_lo;       /* first chunk launched (a shared-prefix pass wrote those below) */
    float qscale;            /* log2(e) / sqrt(dk) */
    const float *k_new;      /* [rows][nkv][dk] fused append (decode), or null */
    const float *v_new;      /* [rows][nkv][dv] */
    uint32_t avg_len;        /* mean visible positions per row (work-group size) */
};

/* One launch of the MFMA causal-prefill kernel. A work item is one tile of
 * 32*waves query rows (token, head-of-group) of one sequence and kv-head. */
struct PrefillArgs {
    const float *q;          /* [T][nh][dk] packed tokens */
    const float *gate;       /* [T][nh][dv] or null */
    float *out;              /* [T][nh][dv] */
    const uint8_t *pool;
    const int32_t *page_table;
    const int32_t *prefix_pages;
    const SeqDev *seqs;
    const uint32_t *items;   /* prefill: [n_items][8] sequence (~0: empty), kv-head, row tile,
                                first packed token, tokens, position, shared-prefix slots,
                                prefix id (-1: none); GQA decode: [rows] the rows' work order,
                                or null */
    const uint32_t *row_seq; /* decode launches (one wave per item): sequence of each row, or null */
    float *part;             /* shared-prefix decode pass: split-KV partials of chunk 0, or null */
    uint32_t max_chunks;     /*   their stride (AttnArgs::max_chunks) */
    uint32_t tab_cap;        /* prefill: key tiles of the longest work item (its per-work-group tile
                                table in LDS), 0: no table */
    PageGeom pg;
    uint32_t n_items;
    uint32_t nh;
    float qscale;
};

struct AppendArgs {
    const float *k;          /* [rows][nkv][dk] */
    const float *v;          /* [rows][nkv][dv] */
    uint8_t *pool;
    const int32_t *page_table;
    const SeqDev *seqs;
    const uint32_t *row_seq;
    const uint32_t *row_t;
    PageGeom pg;
    uint32_t rows;
};

/* Copy of `count` slots between two page lists (prefix build / attach). */
struct CopyArgs {
    uint8_t *pool;           /* layer 0 base; layers at + l * layer_bytes */
    const int32_t *src_pages;
    const int32_t *dst_pages;
    uint32_t src_slot0, dst_slot0, count, n_layers;
    PageGeom pg;
};

/* Gather / scatter of positions to a contiguous staging buffer (inspection). */
struct StageArgs {
    uint8_t *pool;
    const int32_t *pages_for_slot; /* [count] page id per position */
    const uint32_t *slot_in_page;  /* [count] */
    uint8_t *stage_k, *stage_v;    /* [count][nkv][d] */
    float *stage_ks, *stage_vs;    /* [count][nkv] */
    uint32_t count;
    PageGeom pg;
};

struct FillKvArgs {
    uint8_t *pool;
    const int32_t *page_table;
    const int32_t *prefix_pages;
    const SeqDev *seqs;
    const uint32_t *seq_list;
    uint32_t nseq, n_layers;
    uint64_t seed;
    PageGeom pg;
};

/* One launch of the attention front: the qkv tap convolution, per-head
 * ZC-RMSNorm and RoPE on raw projections (engine/src/nd_model.c:2413-2424).
 * A row is one token of one sequence; the rows of a sequence are contiguous
 * and in token order, so token t reads raw rows row-j for j <= t and the tap
 * history for older positions. */
struct FrontArgs {
    const float *q, *k, *v;        /* raw [rows][dq], [rows][dk], [rows][dv] */
    float *q_out;                  /* [rows][dq] */
    float *k_out, *v_out;          /* [rows][dk], [rows][dv]; null: store into the KV pages */
    float *hist;                   /* [max_seqs][n_layers][taps][dcol] raw history */
    const float *w;                /* this layer's tap weights [taps][dcol] (q | k | v columns) */
    const float *norm;             /* this layer's norm scales [2][qk]: q, then k */
    const float2 *rope;            /* [max_pos][qk/2] (cos, sin) */
    const SeqDev *seqs;
    const uint32_t *row_seq;       /* [rows] or null: identity */
    const uint32_t *row_t;         /* [rows] token index within its sequence, or null: 0 */
    uint8_t *pool;                 /* this layer's pool (store mode) */
    const int32_t *page_table;
    PageGeom pg;
    uint32_t rows, layer, n_layers, taps;
    uint32_t nh, nkv, qk, vd;
    uint32_t hist_write;           /* 1: each row writes its raw projection into the history */
};

/* Tap-history maintenance: copies (or zeroes, src null) of whole per-
 * sequence history blocks, applied in order by the host in batches whose
 * blocks do not overlap. */
struct HistOp {
    float *dst;
    const float *src;
};

/* History write-back after a multi-token front launch: the raw rows of the
 * last `taps` tokens of every sequence go to their slots pos % taps. */
struct HistTailArgs {
    const float *q, *k, *v;
    float *hist;
    const SeqDev *seqs;
    const uint32_t *row_seq, *row_t, *row_n;   /* row_n: tokens of the row's sequence */
    uint32_t rows, layer, n_layers, taps, dq, dk, dv;
};

/* CQ projections (nda_cq.hip). */
struct CqPrepArgs {
    const float *x;          /* [rows][in] */
    float *xh;               /* [rows][in_pad] */
    uint32_t rows, in, in_pad, group;
    float scale;             /* 1 / sqrt(group) */
};

/* Up to CQ_MAX_T tensors sharing one prepared activation (same in, group,
 * bits) in one launch: the grid walks their output tiles in order (64
 * outputs per tile in the GEMM, CQ_LUT_OT in the engine-order kernel). */
constexpr int CQ_MAX_T = 8;
constexpr int CQ_LUT_OT = 256;        /* engine-order kernel: outputs per work-group */
constexpr int CQ_LUT_MAX_IN = 2048;   /* its pair table, in_pad * 32 bytes of LDS, within 64 KiB */
struct CqGemmArgs {
    const float *xh;                    /* [rows][in_pad] prepared activations */
    float *y[CQ_MAX_T];                 /* [rows][out[t]] */
    const uint8_t *packed[CQ_MAX_T];    /* [out][rowbytes] LSB-first index bitstream */
    const uint16_t *norms[CQ_MAX_T];    /* [out][ngroup] fp16 bits */
    const float *cb[CQ_MAX_T];          /* [1 << bits] codebook (H's 1/sqrt(group) is in xh) */
    uint32_t out[CQ_MAX_T];
    uint32_t tile0[CQ_MAX_T + 1];       /* first grid.y tile of each tensor; tile0[nt] = total */
    uint32_t nt;
    uint32_t rows, in_pad, group, ngroup, bits, rowbytes;
};

/* The split-precision form of a prepared activation: xh * 2^rexp[r] as an
 * fp16 pair (a, b) per element, rexp chosen per row so the row's largest
 * |value| lands in [2^14, 2^15), in MFMA operand order: [row / 32][col / 16]
 * [plane a, b][lane (row % 32) + 32 (col % 16 / 8)][col % 8] over rows
 * rounded up to 32. */
struct CqPrepSplitArgs {
    const float *x;          /* [rows][in] */
    _Float16 *xs;            /* the operand blocks */
    int32_t *rexp;           /* [rows] */
    uint32_t rows, in, in_pad, group;
    float scale;             /* 1 / sqrt(group) */
    uint32_t rpw;            /* rows per work-group (set by the launcher) */
};

/* 2-bit tensors, group >= 32: the GEMM on fp16 MFMA from split operands. */
struct CqSplitArgs {
    const _Float16 *xs;
    const int32_t *rexp;
    float *y[CQ_MAX_T];
    const uint32_t *cw[CQ_MAX_T];       /* decode data from cq_split_tables_kernel */
    const uint4 *tab[CQ_MAX_T];
    const int32_t *cexp[CQ_MAX_T];
    uint32_t out[CQ_MAX_T];
    uint32_t tile0[CQ_MAX_T + 1];       /* first tile (of CQ_SPLIT_NT outputs) per tensor */
    uint32_t nt;
    uint32_t rows, in_pad, log2_group;
};
/* One 2-bit tensor's decode data for the split GEMM, built at creation:
 * cw [in_pad / 32][out][2] words, tab [ngroup][out] uint4, cexp [out]. */
struct CqTabArgs {
    const uint8_t *packed;
    const uint16_t *norms;
    const float *cb;
    uint32_t *cw;
    uint4 *tab;
    int32_t *cexp;
    uint32_t out, in_pad, ngroup, rowbytes;
};
#ifndef NDA_CQ_OB
#define NDA_CQ_OB 2
#endif
constexpr int CQ_SPLIT_MT = 128;        /* rows per work-group */
constexpr int CQ_SPLIT_OB = NDA_CQ_OB;  /* 32-output blocks per wave */
constexpr int CQ_SPLIT_NT = 64 * CQ_SPLIT_OB;   /* outputs per work-group */

hipError_t launch_cq_prepare(const CqPrepArgs &a, hipStream_t s);
hipError_t launch_cq_gemm(const CqGemmArgs &a, hipStream_t s);
hipError_t launch_cq_lut2(const CqGemmArgs &a, hipStream_t s);
hipError_t launch_cq_prepare_split(const CqPrepSplitArgs &a, hipStream_t s);
hipError_t launch_cq_gemm_split(const CqSplitArgs &a, hipStream_t s);
hipError_t launch_cq_split_tables(const CqTabArgs &a, hipStream_t s);

/* Geometries with kernels specialised for their head dims (KV element bytes,
 * qk_head_dim, v_head_dim, GQA rep): the engine's archive shape and the MHA
 * 8 x 64 shape. Every other shape the engine accepts (head dims multiples of 4
 * up to 64, rep 1-8) runs on the same kernels instantiated for dims padded to
 * 64, with the true dims read at run time. */
#define NDA_FOR_GEOMETRIES(X) \
    X(2, 64, 64, 1) X(2, 64, 64, 2) X(2, 64, 64, 4) X(2, 64, 64, 6) X(2, 64, 64, 8) \
    X(2, 48, 64, 1) X(2, 48, 64, 2) X(2, 48, 64, 6) \
    X(1, 64, 64, 1) X(1, 64, 64, 2) X(1, 64, 64, 4) X(1, 64, 64, 6) X(1, 64, 64, 8) \
    X(1, 48, 64, 1) X(1, 48, 64, 2) X(1, 48, 64, 6)

/* Kernel geometry key. */
struct Geo {
    int kv_f16;
    int dk, dv, rep;
};

/* Launchers (nda_kernels.hip). Return hipSuccess or the launch error;
 * hipErrorNotSupported for a geometry without an instantiation. */
hipError_t launch_append(const Geo &g, const AppendArgs &a, hipStream_t s);
hipError_t launch_attend(const Geo &g, const AttnArgs &a, hipStream_t s);
hipError_t launch_prefill(const Geo &g, const PrefillArgs &a, int waves, hipStream_t s);
/* Largest prefill tile table (PrefillArgs::tab_cap * 16 bytes) a work-group
 * size can take (dma: tiles loaded straight into LDS, fp16 at qk 64); a
 * launch whose table would be larger runs without one. */
uint32_t pf_tab_max_bytes(int waves, bool dma);
/* GQA decode on MFMA: one wave per (row, kv-head) item, n_items = rows * nkv,
 * items in (row, kv-head) order; a.row_seq as in AttnArgs. */
bool decode_mfma_supported(const Geo &g);
hipError_t launch_decode_mfma(const Geo &g, const PrefillArgs &a, hipStream_t s);
hipError_t launch_combine(const Geo &g, const AttnArgs &a, hipStream_t s);
hipError_t launch_copy(const Geo &g, const CopyArgs &a, hipStream_t s);
hipError_t launch_gather(const Geo &g, const StageArgs &a, hipStream_t s);
hipError_t launch_scatter(const Geo &g, const StageArgs &a, hipStream_t s);
hipError_t launch_fill_kv(const Geo &g, const FillKvArgs &a, hipStream_t s);
hipError_t launch_advance(SeqDev *seqs, const uint32_t *seq_list, uint32_t nseq, uint32_t n, hipStream_t s);
hipError_t launch_fill_normal(void *dst, uint64_t n, int dtype, uint64_t seed, float scale,
                              hipStream_t s);
bool geometry_supported(const Geo &g);   /* any shape the engine accepts */
bool geometry_fast(const Geo &g);        /* one of NDA_FOR_GEOMETRIES */
bool prefill_mfma_supported(const Geo &g);

/* nda_front.hip */
hipError_t launch_front(const Geo &g, const FrontArgs &a, hipStream_t s);
hipError_t launch_hist_tail(const HistTailArgs &a, hipStream_t s);
hipError_t launch_hist_ops(const HistOp *d_ops, uint32_t n_ops, uint64_t block_floats, hipStream_t s);

} // namespace nda
