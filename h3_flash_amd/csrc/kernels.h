// Internal launch interface between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "h3attn.h"

namespace h3a {

// Validated attention launch description. Strides are in elements.
struct AttnParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int64_t q_sb, q_sh;  // batch / head strides of Q
    int64_t k_sb, k_sh;
    int64_t v_sb, v_sh;
    int64_t o_sb, o_sh;
    int64_t lse_sb, lse_sh;
    int32_t q_rs, k_rs, v_rs, o_rs;  // sequence (row) strides, in bytes
    int32_t heads;
    int32_t seqlen_q;  // dense: per-batch lengths; varlen: packed row totals
    int32_t seqlen_k;
    int32_t n_qtiles;  // query tiles per (batch-or-segment, head)
    int32_t n_groups;  // batch (dense) or number of segments (varlen)
    float scale_log2;  // softmax_scale * log2(e)
    const int32_t* cu_q;  // NULL for dense
    const int32_t* cu_k;
    // Key-range split of the last tiles (dense only; split_n == 0: none).
    // Tiles [0, n_full) run whole; tiles [n_full, n_full + split_tiles) run as
    // split_n pieces each, which write normalised bf16 partial O and fp32
    // LSE to ws_o / ws_lse for attn_merge to combine.
    int32_t n_full;
    int32_t split_n;
    int32_t split_tiles;
    uint16_t* ws_o;  // bf16 [split_n * split_tiles][kBM][128], normalised
    float* ws_lse;   // [split_n * split_tiles][kBM]
    // Dynamic tail (queue != NULL): workgroups [0, n_full) run whole tiles;
    // the queue_blocks workgroups after them take piece indices
    // [0, split_n * split_tiles) from *queue, which the launch zeroes, until
    // the pieces run out. NULL: pieces are assigned statically.
    int* queue;
    int32_t queue_blocks;
    // Some view spans 2^31 bytes or more: K / V buffer resources are rebased
    // per window of key tiles.
    int32_t wide;
    // d-major V (launches with a workspace; NULL: V is read as given):
    // attn_vt_kernel writes, per (batch, head), 128 rows of vt_rs bytes with
    // keys contiguous, zero past seqlen_k up to a multiple of 64 keys; in a
    // varlen launch segment s starts at key roundup(its first key, 64) + 64 s,
    // zeros between segments.
    void* vt;
    int64_t vt_sb, vt_sh;  // batch / head strides of vt, in elements
    int32_t vt_rs;         // bytes per head-dim row, a multiple of 128
    // Packed varlen launches with a workspace: a work list built on the
    // device by attn_varlen_plan_kernel (NULL: dispatch order, no split).
    // Workgroups [0, ub_tiles) run the list's whole tiles (ub_tiles bounds
    // the non-empty tiles); plan_cus more take the last round's pieces.
    const int32_t* vplan;    // kPlanWords counts and the tail counter
    const int32_t* vlist;    // tile ids, in run order
    const int32_t* vpieces;  // per piece: list position, chunk | chunks << 2 | (merge slot + 1) << 5
    const int32_t* vmerge;   // per merge slot: list position, pieces
    int32_t* vplan_w;        // the same arrays, written by the planning kernel
    int32_t* vlist_w;
    int32_t* vpieces_w;
    int32_t* vmerge_w;
    int32_t* vscratch;       // 4 * num_segments words of the planning kernel
    int32_t ub_tiles;
    int32_t plan_cus;
    // Packed launches of short segments without a work list (persist_queue
    // != NULL): at most persist_blocks persistent workgroups claim tiles from
    // the counter *persist_queue, which the launch zeroes. NULL: one
    // workgroup per tile.
    int* persist_queue;
    int32_t persist_blocks;
};

// Words of the planned-varlen header (vplan).
enum : int { kPlanTiles = 0, kPlanFull = 1, kPlanPieces = 2, kPlanMerges = 3, kPlanQueue = 4, kPlanWords = 16 };

// How the query tiles of a dense launch are spread over the CUs.
struct SplitPlan {
    int32_t n_full, split_n, split_tiles;
    int32_t queue_blocks;   // > 0: dynamic tail with this many workgroups
    int64_t queue_offset;   // byte offset of the tail counter in the workspace
    int64_t workspace_bytes;
};
// max_workspace bounds the plan's workspace_bytes (fewer pieces, or none).
SplitPlan plan_attn_split(int64_t tiles, int64_t key_tiles, int cus, int64_t max_workspace);

// Bytes of the file-scope device array that serves as the workspace of the
// allocation-free attention entry point, and the lookup of the current
// device's copy (hipGetSymbolAddress, cached per device).
constexpr int64_t kStaticScratchBytes = H3A_NOALLOC_SCRATCH_BYTES;
hipError_t attn_static_scratch(void** ptr);

int attn_fwd_block_m();
// Longest segment (max_seqlen_q) of a persistent packed launch.
int attn_fwd_persist_max_rows();
// Most key-range pieces per tile of a tail, and the workspace bytes of one
// piece's fp32 partial O and LSE.
int attn_fwd_tail_pieces();
int64_t attn_fwd_piece_bytes();
int attn_fwd_block_n();
// Rows one buffer resource of the kernel spans from its base (a query tile, or
// a window of key tiles in the wide form); their bytes must stay below 2^31.
int attn_fwd_window_rows();
// Rows past the end of a view that the narrow form may address (all reads
// there are bounds-checked buffer loads returning zero): a view whose rows
// plus this margin span less than 2^31 bytes takes the narrow form.
int attn_fwd_row_margin();
hipError_t launch_attn_fwd(const AttnParams& p, hipStream_t stream);

// n / d for 0 <= n < 2^31 as (umulhi(n, m) + n) >> s (Granlund-Montgomery).
struct FastDiv {
    uint32_t d, m, s;
};
FastDiv make_fast_div(uint32_t d);
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) { return (__umulhi(n, f.m) + n) >> f.s; }

struct QkNormRopeParams {
    const void* x[2];
    void* y[2];
    const void* w[2];
    float eps[2];
    int64_t x_sb[2], x_ss[2], x_sh[2];
    int64_t y_sb[2], y_ss[2], y_sh[2];
    const float* cos;
    const float* sin;
    int64_t table_stride;
    int64_t rows;  // batch * seqlen * n_tensors * heads, < 2^31
    FastDiv div_heads, div_tensors, div_seqlen;
    int32_t seqlen;
    int32_t heads;
    int32_t n_tensors;  // 1 (q only) or 2 (q and k)
    int32_t head_dim;
    int32_t rotary_dim;
    int32_t w_f32;  // 1: weights are fp32, 0: bf16
    // Grouped output heads: head h of y is stored at
    // (h / hpg) * y_sg + (h % hpg) * y_sh; hpg == heads means ungrouped.
    FastDiv div_hpg;
    int64_t y_sg[2];
    // Optional third tensor copied verbatim (no arithmetic) into the same
    // grouped layout (NULL: none).
    const void* xc;
    void* yc;
    int64_t xc_sb, xc_ss, xc_sh;
    int64_t yc_sb, yc_ss, yc_sh, yc_sg;
};

hipError_t launch_qknorm_rope(const QkNormRopeParams& p, hipStream_t stream);
// Whether launch_qknorm_rope takes the fast (lane-group-per-token) path.
bool qknorm_rope_fast_path(const QkNormRopeParams& p);

// Destination-major q/k/v pack. Byte strides; row_bytes = head_dim * element size.
struct PackQkvParams {
    const void* src[3];
    void* out;
    int64_t s_row[3], s_head[3];
    int64_t rows;
    int32_t row_bytes;
    uint32_t units;          // rows * heads, < 2^31
    FastDiv div_heads, div_hl;  // heads, heads per destination
};
hipError_t launch_pack_qkv(const PackQkvParams& p, bool vec, hipStream_t stream);

// (world, rows, inner) -> (rows, world, inner). Byte strides.
struct MergeHeadsParams {
    const void* x;
    void* out;
    int64_t s_world, s_row;
    int64_t rows;
    int64_t inner_bytes;
    uint32_t vectors;            // rows * world * inner_bytes / 16 (vector path), < 2^31
    FastDiv div_inner, div_world;  // inner_bytes / 16, world
};
hipError_t launch_merge_heads(const MergeHeadsParams& p, bool vec, hipStream_t stream);

// RMSNorm + modulation rows; residual != NULL selects the residual + gate
// variant (x is then the branch). Strides in elements.
struct ModulateParams {
    const void* x;
    const void* residual;
    void* out;
    void* hidden;
    const void* weight;
    const void* gate;
    const void* scale;
    const void* shift;
    const void* index;
    int64_t x_stride, residual_stride, out_stride, hidden_stride;
    int64_t gate_stride, scale_stride, shift_stride;
    int64_t rows, n_index, table_rows;
    int32_t cols;
    int32_t w_f32, table_f32, index_i64;
    float eps;
};
// Widest row the register-resident vector path takes.
int modulate_max_vector_cols();
hipError_t launch_modulate(const ModulateParams& p, bool vec, hipStream_t stream);

struct SwigluParams {
    const void* x;
    void* out;
    int64_t x_stride, out_stride, rows, cols;
};
hipError_t launch_swiglu(const SwigluParams& p, bool vec, hipStream_t stream);

// LSE merge of partial attention results over disjoint key ranges.
constexpr int kMergeMaxParts = 16;
struct AttnMergeParams {
    const void* o_parts[kMergeMaxParts];
    const float* lse_parts[kMergeMaxParts];
    void* o;
    float* lse;
    int64_t po_sb, po_ss, po_sh;  // partial outputs (elements)
    int64_t pl_sb, pl_sh;         // partial LSEs
    int64_t o_sb, o_ss, o_sh;
    int64_t l_sb, l_sh;
    int32_t n_parts;
    int32_t heads, seqlen, head_dim;
    int64_t rows;  // batch * seqlen * heads
    int32_t part_f32, out_f32;
};
hipError_t launch_attn_merge(const AttnMergeParams& p, hipStream_t stream);

// Projection GEMM with the q/k norm + RoPE epilogue. Byte strides. Each
// section is a range of output features with its own weight rows, bias,
// output and epilogue (mode 0: plain, 1: RMSNorm over each 128-feature head,
// norm weight, RoPE).
struct ProjSection {
    const void* w;       // bf16 (n, k), w_rs bytes per row
    const void* bias;    // bf16 (n,) or NULL
    const void* norm_w;  // bf16 (128,) (mode 1)
    void* y;             // bf16 (m, n), y_rs bytes per row
    int64_t w_rs, y_rs;
    int32_t n;           // features, a multiple of 128
    int32_t tiles;       // ceil(n / 256)
    int32_t mode;
    float eps;
};
constexpr int kProjMaxSections = 3;
struct ProjGemmParams {
    const void* x;  // bf16 (m, k), x_rs bytes per row
    int64_t x_rs;
    int32_t m, k;   // k a multiple of proj_gemm_k_multiple()
    int32_t m_tiles, n_tiles;  // n_tiles = sum of the sections' tiles
    int32_t n_sections;
    ProjSection sec[kProjMaxSections];
    const float* cos;  // fp32 (seqlen, table_stride) tables (norm sections with rotary_dim > 0)
    const float* sin;
    int64_t table_stride;
    int32_t rotary_dim;
    int32_t seqlen;  // token m uses table row m % seqlen
    int32_t stage_plain;  // 1: sections without RoPE stage their rows in LDS like the RoPE sections
    // 1: the RoPE epilogue reads cos / sin at every rotated column and takes
    // the partners from the token's other lanes (any even rotary_dim, tables
    // in any form, 4-byte aligned); 0: rotary_dim a multiple of 32 with
    // rotate-half tables, 16-byte aligned, read at their first half only.
    int32_t rope_full_tables;
};
int proj_gemm_tile();
int proj_gemm_k_multiple();  // k must be a multiple of this
hipError_t launch_proj_gemm(const ProjGemmParams& p, hipStream_t stream);

// Clock sample (clock.hip): H3A_CLOCK_RECORDS records of 4 uint64 at out.
hipError_t launch_clock_sample(uint64_t* out, hipStream_t stream);

}  // namespace h3a
