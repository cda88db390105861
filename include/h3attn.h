/*
 * h3attn — C ABI of the MI355X (gfx950) dense attention hot path.
 *
 * Two device entry points replace the two GPU steps of the reference's dense
 * attention path inside each MiniMax H3 DiT block:
 *
 *   h3a_attn_fwd      replaces the FlashAttention-4 call made by the dense-FA4
 *                     adapter, `self.kernel(query, key, value, causal=False)`
 *                     (src/h3_flash/runtime/attention/dense_fa4.py:145, call
 *                     form at :74-80) and the torch SDPA call of the fused and
 *                     packed paths (src/h3_flash/runtime/kernels/transformer.py:191-200,
 *                     src/h3_flash/runtime/parallel/packed_ulysses.py:202-209).
 *   h3a_qknorm_rope   replaces the Triton `fused_qknorm_rope(x, weight, cos,
 *                     sin, eps)` (src/h3_flash/runtime/kernels/fusions.py:268-293,
 *                     kernel :126-175), called once for q and once for k at
 *                     src/h3_flash/runtime/kernels/transformer.py:160-173; here
 *                     both tensors are normalised and rotated in one launch.
 *
 * Three more replace the data movement on either side of the packed-Ulysses
 * exchange (src/h3_flash/runtime/parallel/packed_ulysses.py:85-128):
 *
 *   h3a_pack_qkv          pack_qkv_destination_major / _pack_qkv_kernel
 *                         (src/h3_flash/runtime/parallel/relayout.py:11-49,97-130)
 *   h3a_merge_heads       merge_heads / _merge_heads_kernel (relayout.py:52-67,133-159)
 *   h3a_qknorm_rope_pack  the per-rank sequence fused_qknorm_rope(q),
 *                         fused_qknorm_rope(k), pack_qkv_destination_major(q, k, v)
 *                         (packed_ulysses.py:177-200) as one launch.
 *
 * And three replace the other Triton fusions of the DiT block
 * (src/h3_flash/runtime/kernels/fusions.py):
 *
 *   h3a_rmsnorm_modulate                fused_rmsnorm_modulate (:194-215, kernel :69-96)
 *   h3a_residual_gate_rmsnorm_modulate  fused_residual_gate_rmsnorm_modulate
 *                                       (:218-248, kernel :23-67)
 *   h3a_swiglu                          fused_swiglu (:251-265, kernel :98-123)
 *
 * Conventions
 *   - All tensor pointers are device pointers allocated by the caller; the
 *     library allocates nothing and keeps no per-call state (an attention
 *     workspace, when used, is caller memory too).
 *   - Strides are in elements. The last (head_dim / rotary) dimension must be
 *     contiguous.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream).
 *     Nothing synchronises the host.
 *   - Return value: 0 on success, a negative H3A_E* code otherwise; the
 *     message of the last failure on the calling thread is returned by
 *     h3a_last_error().
 *   - Entry points are re-entrant: arguments travel in per-call structs.
 */
#ifndef H3ATTN_H
#define H3ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; only these symbols export. */
#define H3A_API __attribute__((visibility("default")))

#define H3A_ABI_VERSION 4

#define H3A_OK 0
#define H3A_EINVAL (-1)       /* invalid argument (shape, stride, pointer) */
#define H3A_EUNSUPPORTED (-2) /* valid request the library does not implement */
#define H3A_ELAUNCH (-3)      /* the HIP launch itself failed */

/* dtype codes: norm weights and modulation tables (bf16 / fp32), table indices (int32 / int64) */
#define H3A_DTYPE_BF16 0
#define H3A_DTYPE_F32 1
#define H3A_DTYPE_I32 2
#define H3A_DTYPE_I64 3

/*
 * Dense (or block-diagonal varlen) non-causal attention forward,
 *   O = softmax(softmax_scale * Q K^T) V,   LSE = logsumexp(softmax_scale * Q K^T)
 * per (batch, head). Q/K/V/O are bf16 in BSHD layout (batch, seq, head, dim),
 * head_dim must be 128. LSE is fp32, natural log, laid out (batch, head, seq)
 * with non-negative strides lse_stride[0] (batch), lse_stride[1] (head) and 1
 * (seq), 4-byte aligned; it may be NULL when the caller does not want it.
 *
 * Varlen: when cu_seqlens_q is non-NULL, batch must be 1 and the sequence
 * dimension holds `num_segments` packed segments; segment i owns rows
 * [cu_seqlens_q[i], cu_seqlens_q[i+1]) of Q/O/LSE and rows
 * [cu_seqlens_k[i], cu_seqlens_k[i+1]) of K/V (cu_seqlens_k may equal
 * cu_seqlens_q). Both arrays are int32 device arrays of num_segments+1
 * entries; max_seqlen_q bounds every query segment. Attention is
 * block-diagonal: a query attends only to keys of its own segment.
 *
 * Rows with no key (seqlen_k == 0) produce O = 0 and LSE = -inf.
 *
 * Strides: non-negative multiples of 8 elements, the sequence stride at least
 * head_dim. A (batch, head) view may be of any length (strided views of a
 * packed to_qkv output included), but 576 of its rows must span less than
 * 2^31 bytes: a sequence stride under 1,864,136 elements; larger strides
 * return H3A_EUNSUPPORTED. Views whose rows plus an 896-row margin reach
 * 2^31 bytes run in a form of the kernel that rebases its buffer resources
 * per query tile and as the key loop moves on (each within a 576-row
 * window).
 *
 * Extents: batch and heads below 2^31, seqlen_q and seqlen_k below 2^30, and
 * at most 2^31 - 1 query tiles (256 rows of one head) in all; larger ones
 * return H3A_EUNSUPPORTED (sequence lengths: H3A_EINVAL).
 *
 * Workspace: h3a_attn_fwd_workspace_size(args) bytes of device memory at
 * `workspace` (256-byte aligned, contents on entry irrelevant), used for:
 *   - the split tail: with more query tiles (256 rows of one head) than the
 *     GPU has CUs, the tiles of the last round run as key-range pieces that
 *     workgroups take from a counter in the workspace as CUs free up; with
 *     fewer tiles, when they would keep less than 70% of the CUs busy (B=1
 *     H=4 S=4096: 64 tiles on 256 CUs), they run as statically assigned
 *     pieces. Either way the partial results (normalised bf16 O, fp32 LSE)
 *     are merged by a second kernel on the same stream (the counter is
 *     zeroed by a small kernel first);
 *   - a d-major copy of V (per batch and head, 128 rows of keys padded with
 *     zeros to a multiple of 64), written by a transpose kernel at the start
 *     of the call, from which the attention kernel reads each PV fragment
 *     with one 16-byte LDS read;
 *   - packed varlen: a work list planned on the device from cu_seqlens by a
 *     one-workgroup kernel at the start of the call (non-empty tiles,
 *     longest segments first; the last round's tiles as key-range pieces
 *     taken from a counter, merged as above), and the d-major V with each
 *     segment padded to 64 keys. Any cu_seqlens contents keep every access
 *     in bounds; offsets that do not ascend give undefined rows;
 *   - packed varlen with max_seqlen_q below 4,096: 256 bytes, the tile
 *     counter of a persistent launch (one workgroup per CU claims tile after
 *     tile and issues each next tile's first loads during its current one;
 *     the counter is zeroed by a small kernel first). Results are
 *     bit-identical to one workgroup per tile. When the segment lengths vary
 *     (max_seqlen_q at least 1.6 times seqlen_q / num_segments) and there
 *     are few tiles per CU (heads x (seqlen_q / 256 + num_segments / 2) at
 *     most 3.2 per CU, or 9 with max_seqlen_q of 2,900 or more), such calls
 *     take the planned work list above instead.
 * With a NULL or smaller workspace every tile runs whole on V as given. The
 * results differ only by rounding. Calls sharing one workspace must be
 * ordered (same stream).
 */
typedef struct h3a_attn_args {
    int32_t abi_version; /* must be H3A_ABI_VERSION */
    const void *q;       /* bf16 */
    const void *k;       /* bf16 */
    const void *v;       /* bf16 */
    void *o;             /* bf16 */
    float *lse;          /* fp32 or NULL */
    int64_t batch;
    int64_t heads;
    int64_t seqlen_q;
    int64_t seqlen_k;
    int64_t head_dim;
    int64_t q_stride[3]; /* batch, seq, head */
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int64_t lse_stride[2]; /* batch, head */
    float softmax_scale;
    int32_t causal; /* must be 0: the path is non-causal */
    const int32_t *cu_seqlens_q;
    const int32_t *cu_seqlens_k;
    int32_t num_segments;
    int32_t max_seqlen_q;
    void *workspace;         /* device memory or NULL, see above */
    int64_t workspace_bytes; /* bytes available at workspace */
} h3a_attn_args;

H3A_API int h3a_attn_fwd(const h3a_attn_args *args, void *stream);

/*
 * Bytes of workspace h3a_attn_fwd can use for these arguments on the current
 * device (0: none); a negative H3A_E* code when the arguments are invalid.
 * No counterpart in the reference: FlashAttention sizes its own scratch.
 */
H3A_API int64_t h3a_attn_fwd_workspace_size(const h3a_attn_args *args);

/*
 * h3a_attn_fwd without allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory per call (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, semantics and results (up to the rounding of the key-range
 * pieces) as h3a_attn_fwd; `workspace` / `workspace_bytes` are ignored. The
 * split tail's partial results (bf16 O, fp32 LSE) and counter live in a file-scope device
 * array of H3A_NOALLOC_SCRATCH_BYTES (64 MiB) that every GPU the library
 * runs on holds until the process ends; its address is looked up once per
 * device. The split plan is fitted to that array (fewer key-range pieces,
 * or none), so any problem size runs; a plan that could not be fitted would
 * be rejected with H3A_EINVAL. Packed calls with max_seqlen_q below 4,096
 * run the persistent launch, its tile counter in the same array (also those
 * of varied lengths, whose planned list would not fit). The call allocates
 * nothing, issues no memset and does not synchronise.
 *
 * All calls on one GPU share its array: calls that overlap on one GPU (on
 * different streams, or from different threads without ordering) race on
 * it and give wrong results. Order them on one stream.
 */
#define H3A_NOALLOC_SCRATCH_BYTES ((int64_t)64 << 20)
H3A_API int h3a_attn_fwd_noalloc(const h3a_attn_args *args, void *stream);

/*
 * Fused per-head RMSNorm + rotate-half RoPE on q and k in one launch:
 *   r      = rsqrt(mean(x^2) + eps)            (over head_dim, fp32)
 *   n[c]   = x[c] * r * w[c]
 *   y[c]   = n[c]*cos[s,c] - n[c+R/2]*sin[s,c]   c <  R/2
 *   y[c]   = n[c]*cos[s,c] + n[c-R/2]*sin[s,c]   R/2 <= c < R
 *   y[c]   = n[c]                               c >= R
 * stored in bf16. x/y are bf16 in BSHD layout; w is (head_dim,) in bf16 or
 * fp32 (w_dtype); cos/sin are fp32 (seqlen, R) tables with row stride
 * table_stride. R must be even and <= head_dim; head_dim a multiple of 8 and
 * at most 512. xk/yk/wk may be NULL to transform one tensor only. y may alias
 * x (in place).
 */
typedef struct h3a_qknorm_rope_args {
    int32_t abi_version;
    const void *xq;
    const void *xk;
    void *yq;
    void *yk;
    const void *wq;
    const void *wk;
    int32_t w_dtype;
    const float *cos;
    const float *sin;
    int64_t table_stride;
    int64_t batch;
    int64_t seqlen;
    int64_t heads;
    int64_t head_dim;
    int64_t rotary_dim;
    int64_t xq_stride[3]; /* batch, seq, head */
    int64_t xk_stride[3];
    int64_t yq_stride[3];
    int64_t yk_stride[3];
    float eps_q;
    float eps_k;
} h3a_qknorm_rope_args;

H3A_API int h3a_qknorm_rope(const h3a_qknorm_rope_args *args, void *stream);

/*
 * Destination-major pack of q, k, v for the packed-Ulysses QKV exchange:
 *   out[dest][row][lh][i*head_dim + d] = X_i[row][dest*hl + lh][d]
 * with X = (q, k, v), hl = heads / world, and out contiguous of shape
 * (world, rows, hl, 3*head_dim). Elements of elem_bytes (1, 2, 4 or 8) bytes
 * are moved, never converted. q/k/v are (rows, heads, head_dim) with element
 * strides {row, head} and a contiguous last dimension. heads must be a
 * multiple of world (H3A_EINVAL otherwise, with the reference's message).
 */
typedef struct h3a_pack_qkv_args {
    int32_t abi_version;
    const void *q;
    const void *k;
    const void *v;
    void *out;
    int64_t elem_bytes;
    int64_t rows;
    int64_t heads;
    int64_t head_dim;
    int64_t world;
    int64_t q_stride[2]; /* row, head */
    int64_t k_stride[2];
    int64_t v_stride[2];
} h3a_pack_qkv_args;

H3A_API int h3a_pack_qkv(const h3a_pack_qkv_args *args, void *stream);

/*
 * Source-rank / row transpose after the output exchange:
 *   out[row][src][t] = x[src][row][t],  t < inner (= heads_local * head_dim)
 * x has element strides {world, row} and a contiguous inner dimension; out is
 * contiguous (rows, world, inner). Elements are moved, never converted.
 */
typedef struct h3a_merge_heads_args {
    int32_t abi_version;
    const void *x;
    void *out;
    int64_t elem_bytes;
    int64_t world;
    int64_t rows;
    int64_t inner;
    int64_t x_stride[2]; /* world, row */
} h3a_merge_heads_args;

H3A_API int h3a_merge_heads(const h3a_merge_heads_args *args, void *stream);

/*
 * h3a_qknorm_rope on q and k plus h3a_pack_qkv in one launch: q and k
 * ((rows, heads, head_dim) bf16, strides {row, head}) are normalised and
 * rotated exactly as by h3a_qknorm_rope (same arithmetic, same rounding) and
 * written, with v copied verbatim, into the destination-major buffer `out`
 * of h3a_pack_qkv. Batch is 1 (the packed path's only case). Any even
 * rotary width up to head_dim, as for h3a_qknorm_rope; cos/sin 4-byte
 * aligned (a rotary width that is a multiple of 16 with 16-byte aligned
 * table rows takes the vectorised kernel, others an element-wise one with
 * the same results).
 */
typedef struct h3a_qknorm_rope_pack_args {
    int32_t abi_version;
    const void *q;
    const void *k;
    const void *v;
    void *out;
    const void *wq;
    const void *wk;
    int32_t w_dtype;
    const float *cos;
    const float *sin;
    int64_t table_stride;
    int64_t rows;
    int64_t heads;
    int64_t head_dim;
    int64_t rotary_dim;
    int64_t world;
    int64_t q_stride[2]; /* row, head */
    int64_t k_stride[2];
    int64_t v_stride[2];
    float eps_q;
    float eps_k;
} h3a_qknorm_rope_pack_args;

H3A_API int h3a_qknorm_rope_pack(const h3a_qknorm_rope_pack_args *args, void *stream);

/*
 * Per row r (token) with modulation-table row t = index[r % n_index]:
 *   n      = x[r] * rsqrt(sum(x[r]^2) / cols + eps)
 *   out[r] = n * weight * (1 + scale[t]) + shift[t]
 * in fp32, stored once in bf16. x/out are bf16 (rows, cols) with row strides
 * in elements; weight is (cols,) bf16 or fp32 (w_dtype); scale and shift are
 * (table_rows, cols) bf16 or fp32 (table_dtype) with their own row strides;
 * index is int32 or int64 (index_dtype). Indices outside [0, table_rows) are
 * clamped to the table.
 */
typedef struct h3a_rmsnorm_modulate_args {
    int32_t abi_version;
    const void *x;
    void *out;
    const void *weight;
    int32_t w_dtype;
    const void *scale;
    const void *shift;
    int32_t table_dtype;
    int64_t scale_stride;
    int64_t shift_stride;
    int64_t table_rows;
    const void *index;
    int32_t index_dtype;
    int64_t n_index;
    int64_t rows;
    int64_t cols;
    int64_t x_stride;
    int64_t out_stride;
    float eps;
} h3a_rmsnorm_modulate_args;

H3A_API int h3a_rmsnorm_modulate(const h3a_rmsnorm_modulate_args *args, void *stream);

/*
 * Per row r with t = index[r % n_index]:
 *   h             = residual[r] + gate[t] * branch[r]        (fp32)
 *   hidden_out[r] = h                                        (bf16)
 *   n             = h * rsqrt(sum(h^2) / cols + eps) * weight
 *   normed_out[r] = n * (1 + scale[t]) + shift[t]            (bf16)
 * The norm uses the unrounded fp32 h. Layouts and dtypes as for
 * h3a_rmsnorm_modulate; gate is a (table_rows, cols) table like scale.
 */
typedef struct h3a_residual_gate_rmsnorm_modulate_args {
    int32_t abi_version;
    const void *residual;
    const void *branch;
    void *hidden_out;
    void *normed_out;
    const void *weight;
    int32_t w_dtype;
    const void *gate;
    const void *scale;
    const void *shift;
    int32_t table_dtype;
    int64_t gate_stride;
    int64_t scale_stride;
    int64_t shift_stride;
    int64_t table_rows;
    const void *index;
    int32_t index_dtype;
    int64_t n_index;
    int64_t rows;
    int64_t cols;
    int64_t residual_stride;
    int64_t branch_stride;
    int64_t hidden_stride;
    int64_t normed_stride;
    float eps;
} h3a_residual_gate_rmsnorm_modulate_args;

H3A_API int h3a_residual_gate_rmsnorm_modulate(const h3a_residual_gate_rmsnorm_modulate_args *args, void *stream);

/*
 * out[r, c] = x[r, c] * (g * sigmoid(g)),  g = x[r, cols + c]
 * x is bf16 (rows, 2*cols), out bf16 (rows, cols); row strides in elements.
 */
typedef struct h3a_swiglu_args {
    int32_t abi_version;
    const void *x;
    void *out;
    int64_t rows;
    int64_t cols;
    int64_t x_stride;
    int64_t out_stride;
} h3a_swiglu_args;

H3A_API int h3a_swiglu(const h3a_swiglu_args *args, void *stream);

/*
 * Merge of partial attention results over disjoint key ranges, the combine
 * step of ring / context-parallel attention over the (out, lse) pairs that
 * h3a_attn_fwd returns per key chunk:
 *   lse = log(sum_p exp(lse_p)),   out = sum_p exp(lse_p - lse) * out_p
 * in fp32. Parts with lse = -inf weigh nothing; a row with no keys in any
 * part gets out = 0 and lse = -inf. Partial outputs share one BSHD layout
 * (part_o_stride) and dtype (bf16 or fp32); partial LSEs share one (B, H, S)
 * layout. out (bf16 or fp32) and lse may alias part 0 (in-place online
 * merge). 1 <= n_parts <= 16; head_dim a multiple of 8, at most 512; every
 * row 16-byte aligned; LSE pointers 4-byte aligned, all strides non-negative.
 * No counterpart in the reference's kernels: the FA4 adapter cannot return
 * the LSE (dense_fa4.py:72-73); this is what a context-parallel forward op
 * with return_lse=True (dense_fa4.py:53-81) is merged with.
 */
#define H3A_MERGE_MAX_PARTS 16

typedef struct h3a_attn_merge_args {
    int32_t abi_version;
    int32_t n_parts;
    const void *o_parts[H3A_MERGE_MAX_PARTS];
    const float *lse_parts[H3A_MERGE_MAX_PARTS];
    int32_t part_dtype; /* H3A_DTYPE_BF16 or H3A_DTYPE_F32 */
    void *o;
    int32_t out_dtype;  /* H3A_DTYPE_BF16 or H3A_DTYPE_F32 */
    float *lse;         /* may be NULL */
    int64_t batch;
    int64_t heads;
    int64_t seqlen;
    int64_t head_dim;
    int64_t part_o_stride[3];   /* batch, seq, head */
    int64_t part_lse_stride[2]; /* batch, head */
    int64_t o_stride[3];
    int64_t lse_stride[2];
} h3a_attn_merge_args;

H3A_API int h3a_attn_merge(const h3a_attn_merge_args *args, void *stream);

/*
 * Projection GEMM of an H3 attention block with the q/k prologue as its
 * epilogue. For every token row m of x and output feature f of a section,
 *   acc = sum_k x[m, k] * weight[f, k] + bias[f]        (fp32 accumulation)
 * and then per section mode:
 *   H3A_PROJ_PLAIN:        y[m, f] = bf16(acc)
 *   H3A_PROJ_QKNORM_ROPE:  per head (128 consecutive features) of token m,
 *     with p = bf16(acc) (the projection as the module's linear outputs it),
 *     n = p * rsqrt(sum(p^2) / 128 + eps) * norm_weight[f mod 128], then
 *     rotate-half RoPE over the head's first rotary_dim features with table
 *     row s = m mod seqlen:
 *       y[c] = n[c] cos[s,c] - n[c+R/2] sin[s,c]   (c < R/2)
 *       y[c] = n[c] cos[s,c] + n[c-R/2] sin[s,c]   (R/2 <= c < R)
 *       y[c] = n[c]                                (c >= R)
 *     in fp32, stored as bf16 (rotary_dim 0: the norm alone).
 * This is the reference's projection step followed by its fused q/k norm +
 * RoPE, in the reference's rounding order (the projection rounded to bf16,
 * then the norm and RoPE computed in fp32 and rounded once more):
 *   attn.to_qkv(hidden_states).chunk(3) or to_q / to_k / to_v
 *     (src/h3_flash/runtime/attention/dense_fa4.py:123-128,
 *      src/h3_flash/runtime/kernels/transformer.py:146-152),
 *   norm_q / norm_k and _apply_rotary_emb, or fused_qknorm_rope
 *     (dense_fa4.py:132-140, transformer.py:155-173, fusions.py:268-293),
 *   and attn.to_out[0] (dense_fa4.py:169) as one PLAIN section.
 * x: bf16 (m, k) with row stride x_stride elements; weight: bf16 (n, k) rows
 * (the nn.Linear layout); y: bf16 (m, n) with row stride y_stride. Up to three
 * sections (q, k, v of one fused or three separate weights) share x and run in
 * one launch. head_dim must be 128; k a positive multiple of 128; each n a
 * positive multiple of 128; x, weight and y 16-byte aligned with strides that
 * are multiples of 8 elements; bias and norm_weight (bf16) 8-byte aligned;
 * rotary_dim any even width up to 128 (as fused_qknorm_rope takes,
 * fusions.py:268-275); cos / sin fp32 (seqlen rows of table_stride >=
 * rotary_dim floats), 4-byte aligned. With rotary_dim a multiple of 32,
 * rotate_half_tables = 1 and 16-byte aligned table rows (table_stride a
 * multiple of 4), each lane holds its RoPE partners and only the tables'
 * first half is read; otherwise the partners come from the token's other
 * lanes through LDS and the tables are read at every rotated column (same
 * results). No workspace; nothing is allocated.
 */
#define H3A_PROJ_PLAIN 0
#define H3A_PROJ_QKNORM_ROPE 1
#define H3A_PROJ_MAX_SECTIONS 3

typedef struct h3a_proj_section {
    const void *weight;      /* bf16 (n, k) */
    int64_t weight_stride;   /* elements between weight rows */
    int64_t n;               /* output features */
    const void *bias;        /* bf16 (n,) or NULL */
    void *y;                 /* bf16 (m, n) */
    int64_t y_stride;        /* elements between y rows */
    int32_t mode;            /* H3A_PROJ_PLAIN or H3A_PROJ_QKNORM_ROPE */
    const void *norm_weight; /* bf16 (head_dim,), H3A_PROJ_QKNORM_ROPE only */
    float eps;
} h3a_proj_section;

typedef struct h3a_proj_args {
    int32_t abi_version;
    const void *x;      /* bf16 (m, k) */
    int64_t x_stride;   /* elements between x rows */
    int64_t m;
    int64_t k;
    int64_t head_dim;   /* 128 */
    int32_t num_sections;
    h3a_proj_section sections[H3A_PROJ_MAX_SECTIONS];
    const float *cos;   /* fp32 (seqlen, table_stride), or NULL when rotary_dim is 0 */
    const float *sin;
    int64_t table_stride;
    int64_t rotary_dim; /* even, 0 .. 128 */
    int64_t seqlen;     /* table rows; token row m uses row m % seqlen */
    int32_t rotate_half_tables; /* 1: the caller guarantees cos[:, c] == cos[:, c + R/2] and
                                   sin[:, c] == sin[:, c + R/2] (the cat(theta, theta) form of
                                   rotate-half RoPE tables), which lets a rotary_dim that is a
                                   multiple of 32 read the first R/2 columns only; 0: tables of
                                   any form, read at every rotated column */
} h3a_proj_args;

H3A_API int h3a_proj_gemm(const h3a_proj_args *args, void *stream);

/*
 * Device clock sample. A measurement aid with no counterpart in the reference
 * (its benchmark, benchmarks/benchmark_dense_fa4.py:84-136, reports wall time
 * only); for benchmarks that quote a fraction of the nominal MFMA peak, which
 * depends on the core clock the part holds under load.
 *
 * Launches H3A_CLOCK_RECORDS one-wave workgroups on `stream`, enough for
 * every CU to run several. Workgroup i writes four values to
 * out[4*i .. 4*i+3] (a device array of 4 * H3A_CLOCK_RECORDS uint64):
 *   the XCD it ran on (HW_REG_XCC_ID), its hardware wave id (HW_REG_HW_ID:
 *   bits 8-15 name the CU within the XCD), the CU's shader clock counter
 *   (s_memtime, core clock cycles) and the chip's constant 100 MHz realtime
 *   counter (s_memrealtime).
 * The cycle counters of different CUs are not aligned with each other, and
 * a CU's counter advances only while the CU is clocked. Two samples on one
 * stream around a stretch of work that keeps every CU busy give each CU's
 * mean core clock over it, from the records of the same (XCD, CU) in both:
 * 100 MHz * d(memtime) / d(realtime).
 */
#define H3A_CLOCK_RECORDS 2048
H3A_API int h3a_clock_sample(uint64_t *out, void *stream);

/* Message of the last failed call on this thread ("" if none). */
H3A_API const char *h3a_last_error(void);

/* H3A_ABI_VERSION of the loaded library. */
H3A_API int h3a_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* H3ATTN_H */
