// extern "C" entry points declared in include/h3attn.h: argument validation,
// error reporting and launch of the gfx950 kernels. No allocation, no host
// synchronisation, no global mutable state besides the per-thread message and
// a per-device cache of the CU count.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "h3attn.h"
#include "kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

constexpr int64_t kMaxWindow = (int64_t)1 << 31;  // buffer offsets are 32-bit
// The d-major V copy costs a pass over V (about 25 us at 5 heads x 49,920
// keys) and saves about 1.9% of the attention: it pays from about 14k keys
// per sequence (segment) on; below that V is read as given.
constexpr int64_t kVtMinKeys = 16384;
// A planned varlen launch (device-built work list with a balanced last
// round) pays for its planning launch with segments of this many rows.
constexpr int64_t kPlanMinSegment = 4096;

// Shorter segments run on the persistent launch, unless their lengths vary
// and there are few tiles per CU: its last tiles (up to max_seqlen_q / 64
// key tiles each, claimed in segment order) then leave CUs idle, and each
// tile past a shorter segment's rows costs a claim. The planned list (no
// such tiles, longest segments first, the last round as key-range pieces)
// balances them. Equal lengths and many rounds keep the persistent launch
// (its next-tile loads). Timed on 47 mixes of H5 segments of 1 to 4,095
// rows, this rule picked the faster launch for all but three, each within
// 4% of it. The host knows only the packed rows, the segment count and the
// longest segment, so "varied" is the longest against the mean.
bool short_segments_planned(const h3a_attn_args* a, int cus) {
    if (a->num_segments <= 0 || a->seqlen_q <= 0 || cus <= 0) return false;
    const double mean = (double)a->seqlen_q / (double)a->num_segments;
    const double rounds =
        (double)a->heads * ((double)a->seqlen_q / h3a::attn_fwd_block_m() + a->num_segments / 2.0) / cus;
    const bool varied = a->max_seqlen_q >= 1.6 * mean;
    return varied && (rounds <= 3.2 || (a->max_seqlen_q >= 2900 && rounds <= 9.0));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }

// Validates the arguments and fills the launch description (split off);
// *empty: nothing to launch.
int prepare_attn(const h3a_attn_args* a, h3a::AttnParams& p, bool* empty) {
    *empty = false;
    if (a == nullptr) return fail(H3A_EINVAL, "h3a_attn_fwd: args is NULL");
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "h3a_attn_fwd: abi_version %d, library is %d", a->abi_version, H3A_ABI_VERSION);
    if (a->causal != 0) return fail(H3A_EUNSUPPORTED, "h3a_attn_fwd: causal attention is not supported (non-causal path)");
    if (a->head_dim != 128) return fail(H3A_EUNSUPPORTED, "h3a_attn_fwd: head_dim must be 128, got %lld", (long long)a->head_dim);
    if (a->batch < 0 || a->heads <= 0 || a->seqlen_q < 0 || a->seqlen_k < 0)
        return fail(H3A_EINVAL, "h3a_attn_fwd: negative or zero extent (batch=%lld heads=%lld sq=%lld sk=%lld)",
                    (long long)a->batch, (long long)a->heads, (long long)a->seqlen_q, (long long)a->seqlen_k);
    if (!(a->softmax_scale > 0.f) || !isfinite(a->softmax_scale))
        return fail(H3A_EINVAL, "h3a_attn_fwd: softmax_scale must be finite and > 0");
    // The launch description holds these in 32 bits.
    if (a->batch > INT32_MAX || a->heads > INT32_MAX)
        return fail(H3A_EUNSUPPORTED, "h3a_attn_fwd: batch and heads must be below 2^31");
    if (a->batch == 0 || a->seqlen_q == 0) {
        *empty = true;
        return H3A_OK;
    }
    if (!a->q || !a->o || (a->seqlen_k > 0 && (!a->k || !a->v)))
        return fail(H3A_EINVAL, "h3a_attn_fwd: NULL tensor pointer");
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o))
        return fail(H3A_EINVAL, "h3a_attn_fwd: q/k/v/o must be 16-byte aligned");
    if (a->lse != nullptr && (!aligned4(a->lse) || a->lse_stride[0] < 0 || a->lse_stride[1] < 0))
        return fail(H3A_EINVAL, "h3a_attn_fwd: lse must be 4-byte aligned with non-negative strides");
    const int64_t* st[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
    const char* nm[4] = {"q", "k", "v", "o"};
    for (int i = 0; i < 4; ++i) {
        for (int d = 0; d < 3; ++d)
            if (st[i][d] < 0 || st[i][d] % 8 != 0)
                return fail(H3A_EINVAL, "h3a_attn_fwd: %s strides must be non-negative multiples of 8 elements", nm[i]);
        if (st[i][1] < 128) return fail(H3A_EINVAL, "h3a_attn_fwd: %s sequence stride %lld < head_dim", nm[i], (long long)st[i][1]);
    }

    const bool varlen = a->cu_seqlens_q != nullptr;
    p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o; p.lse = a->lse;
    p.q_sb = a->q_stride[0]; p.q_sh = a->q_stride[2];
    p.k_sb = a->k_stride[0]; p.k_sh = a->k_stride[2];
    p.v_sb = a->v_stride[0]; p.v_sh = a->v_stride[2];
    p.o_sb = a->o_stride[0]; p.o_sh = a->o_stride[2];
    p.lse_sb = a->lse_stride[0]; p.lse_sh = a->lse_stride[1];
    p.heads = (int32_t)a->heads;
    p.scale_log2 = a->softmax_scale * 1.4426950408889634f;
    const int bm = h3a::attn_fwd_block_m();
    if (varlen) {
        if (a->cu_seqlens_k == nullptr) return fail(H3A_EINVAL, "h3a_attn_fwd: cu_seqlens_q given without cu_seqlens_k");
        if (a->batch != 1) return fail(H3A_EINVAL, "h3a_attn_fwd: varlen requires batch == 1, got %lld", (long long)a->batch);
        if (a->num_segments <= 0) return fail(H3A_EINVAL, "h3a_attn_fwd: num_segments must be > 0");
        if (a->max_seqlen_q <= 0 || a->max_seqlen_q > a->seqlen_q)
            return fail(H3A_EINVAL, "h3a_attn_fwd: max_seqlen_q must be in [1, seqlen_q]");
        p.cu_q = a->cu_seqlens_q;
        p.cu_k = a->cu_seqlens_k;
        p.n_groups = a->num_segments;
        p.n_qtiles = (a->max_seqlen_q + bm - 1) / bm;
        if (a->seqlen_q > INT32_MAX / 2 || a->seqlen_k > INT32_MAX / 2)
            return fail(H3A_EINVAL, "h3a_attn_fwd: sequence length too large");
        p.seqlen_q = (int32_t)a->seqlen_q;  // packed totals; segments are clamped to them
        p.seqlen_k = (int32_t)a->seqlen_k;
    } else {
        if (a->seqlen_q > INT32_MAX / 2 || a->seqlen_k > INT32_MAX / 2)
            return fail(H3A_EINVAL, "h3a_attn_fwd: sequence length too large");
        p.cu_q = nullptr; p.cu_k = nullptr;
        p.n_groups = (int32_t)a->batch;
        p.n_qtiles = (int32_t)((a->seqlen_q + bm - 1) / bm);
        p.seqlen_q = (int32_t)a->seqlen_q;
        p.seqlen_k = (int32_t)a->seqlen_k;
    }
    // The kernel addresses a view through buffer resources rebased to each
    // query tile and each window of key tiles, with 32-bit byte offsets
    // inside them: a view may be of any length, but attn_fwd_window_rows()
    // rows of it must span less than 2^31 bytes.
    const int64_t window = h3a::attn_fwd_window_rows();
    for (int i = 0; i < 4; ++i) {
        // window * stride * 2 >= kMaxWindow, without overflowing int64
        if (st[i][1] >= (kMaxWindow + window * 2 - 1) / (window * 2))
            return fail(H3A_EUNSUPPORTED, "h3a_attn_fwd: %s row stride %lld elements is too large (%lld rows must span < 2^31 bytes)",
                        nm[i], (long long)st[i][1], (long long)window);
    }
    // Views short enough for one buffer resource each (rows plus the
    // kernel's margin under 2^31 bytes) take the narrow form.
    const int64_t rows[4] = {a->seqlen_q, a->seqlen_k, a->seqlen_k, a->seqlen_q};
    p.wide = 0;
    for (int i = 0; i < 4; ++i)
        if ((rows[i] + h3a::attn_fwd_row_margin()) * st[i][1] * 2 >= kMaxWindow) p.wide = 1;
    p.q_rs = (int32_t)(a->q_stride[1] * 2);
    p.k_rs = (int32_t)(a->k_stride[1] * 2);
    p.v_rs = (int32_t)(a->v_stride[1] * 2);
    p.o_rs = (int32_t)(a->o_stride[1] * 2);
    const int64_t blocks = (int64_t)p.n_qtiles * p.heads * p.n_groups;
    if (blocks > INT32_MAX) return fail(H3A_EUNSUPPORTED, "h3a_attn_fwd: grid too large");
    return H3A_OK;
}

// CU count of the current device, cached per device.
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Split plan of a validated launch: dense inputs only (varlen tiles are not
// uniform work).
h3a::SplitPlan attn_plan(const h3a_attn_args* a, const h3a::AttnParams& p, int64_t max_workspace = INT64_MAX) {
    const int64_t tiles = (int64_t)p.n_qtiles * p.heads * p.n_groups;
    h3a::SplitPlan none{(int32_t)tiles, 0, 0, 0, 0, 0};
    if (a->cu_seqlens_q != nullptr) return none;
    const int bn = h3a::attn_fwd_block_n();
    return h3a::plan_attn_split(tiles, (a->seqlen_k + bn - 1) / bn, device_cus(), max_workspace);
}

// The workspace of a launch: the split plan's partial results and counter,
// then (dense launches, allow_vt) a d-major copy of V, 128 rows of keys per
// (batch, head) padded to a multiple of 64 keys.
struct AttnWorkspace {
    h3a::SplitPlan plan;
    int64_t vt_offset;  // 0: no d-major V
    int64_t vt_rs;      // bytes per row of keys (0: no d-major V)
    // Packed varlen with a device-built work list (ub_tiles > 0): partial
    // results at 0, the plan's words at plan_offset.
    int64_t plan_offset;
    int32_t ub_tiles, cus;
    int64_t total;
    bool persist;  // short packed segments: a tile counter at offset 0
};

AttnWorkspace attn_workspace(const h3a_attn_args* a, const h3a::AttnParams& p, bool allow_vt,
                             int64_t max_workspace = INT64_MAX) {
    AttnWorkspace w{attn_plan(a, p, max_workspace), 0, 0, 0, 0, 0, 0, false};
    w.total = w.plan.workspace_bytes;
    const int bn = h3a::attn_fwd_block_n();
    if (a->cu_seqlens_q != nullptr) {
        // Packed varlen: the work list, the last round's partial results (at
        // most tail_pieces per CU-round tile), and a d-major V whose segments
        // are each padded to a multiple of 64 keys.
        // Only for segments long enough that a balanced last round pays for
        // the planning launch (max_seqlen_q bounds them).
        const int cus = device_cus();
        if (!allow_vt || cus <= 0) return w;
        if (a->max_seqlen_q < kPlanMinSegment && !short_segments_planned(a, cus)) {
            // Short segments: the persistent launch's tile counter.
            if (a->max_seqlen_q <= h3a::attn_fwd_persist_max_rows() && w.total + 256 <= max_workspace) {
                w.persist = true;
                w.cus = cus;
                w.total += 256;
            }
            return w;
        }
        const int64_t nseg = a->num_segments, bm = h3a::attn_fwd_block_m();
        const int64_t grid = (int64_t)p.n_qtiles * p.heads * p.n_groups;
        int64_t ub = a->heads * ((a->seqlen_q + bm - 1) / bm + nseg);
        ub = ub < grid ? ub : grid;
        const int64_t pieces = (int64_t)h3a::attn_fwd_tail_pieces() * cus;
        const int64_t words = h3a::kPlanWords + ub + 2 * pieces + 2 * cus + 4 * nseg;
        w.plan_offset = pieces * h3a::attn_fwd_piece_bytes();
        w.total = w.plan_offset + (4 * words + 255) / 256 * 256;
        if (w.total > max_workspace) return AttnWorkspace{w.plan, 0, 0, 0, 0, 0, 0, false};
        w.ub_tiles = (int32_t)ub;
        w.cus = cus;
        const int64_t vt_rs = ((a->seqlen_k + bn - 1) / bn * bn + bn * nseg) * 2;
        if (a->seqlen_k == 0 || a->max_seqlen_q < kVtMinKeys || 128 * vt_rs >= kMaxWindow) return w;
        const int64_t bytes = a->heads * 128 * vt_rs;
        if (w.total + bytes > max_workspace) return w;
        w.vt_offset = w.total;
        w.vt_rs = vt_rs;
        w.total += bytes;
        return w;
    }
    const int64_t vt_rs = (a->seqlen_k + bn - 1) / bn * bn * 2;
    // The d-major V is addressed with 32-bit offsets within a head's block.
    if (!allow_vt || a->seqlen_k < kVtMinKeys || 128 * vt_rs >= kMaxWindow) return w;
    const int64_t offset = (w.total + 255) / 256 * 256;
    const int64_t bytes = a->batch * a->heads * 128 * vt_rs;
    if (offset + bytes > max_workspace) return w;
    w.vt_offset = offset;
    w.vt_rs = vt_rs;
    w.total = offset + bytes;
    return w;
}

// Points the launch at a workspace for the plan's split tiles.
void apply_plan(h3a::AttnParams& p, const h3a::SplitPlan& plan, void* workspace) {
    p.n_full = plan.n_full;
    p.split_n = plan.split_n;
    p.split_tiles = plan.split_tiles;
    p.ws_o = (uint16_t*)workspace;
    p.ws_lse = (float*)(p.ws_o + (int64_t)plan.split_n * plan.split_tiles * h3a::attn_fwd_block_m() * 128);
    if (plan.queue_blocks > 0) {
        p.queue = (int*)((char*)workspace + plan.queue_offset);
        p.queue_blocks = plan.queue_blocks;
    }
}

// Shared checks of the modulation entry points. Fills the table, index and
// weight fields of p and reports whether the 16-byte vector path applies to
// them (activations are checked by the caller).
int prepare_modulate(const char* fn, const void* weight, int32_t w_dtype, const void* const* tables,
                     const int64_t* table_strides, int n_tables, int32_t table_dtype, int64_t table_rows,
                     const void* index, int32_t index_dtype, int64_t n_index, int64_t rows, int64_t cols, float eps,
                     h3a::ModulateParams& p, bool* vec) {
    if (rows < 0 || cols <= 0 || cols >= ((int64_t)1 << 31) || rows >= ((int64_t)1 << 31))
        return fail(H3A_EINVAL, "%s: bad extents (rows=%lld cols=%lld)", fn, (long long)rows, (long long)cols);
    if (w_dtype != H3A_DTYPE_BF16 && w_dtype != H3A_DTYPE_F32) return fail(H3A_EINVAL, "%s: unknown weight dtype %d", fn, w_dtype);
    if (table_dtype != H3A_DTYPE_BF16 && table_dtype != H3A_DTYPE_F32)
        return fail(H3A_EINVAL, "%s: unknown table dtype %d", fn, table_dtype);
    if (index_dtype != H3A_DTYPE_I32 && index_dtype != H3A_DTYPE_I64)
        return fail(H3A_EINVAL, "%s: index dtype must be int32 or int64, got code %d", fn, index_dtype);
    if (n_index <= 0 || table_rows <= 0) return fail(H3A_EINVAL, "%s: n_index and table_rows must be > 0", fn);
    if (!(eps >= 0.f)) return fail(H3A_EINVAL, "%s: eps must be >= 0", fn);
    if (rows > 0 && (!weight || !index)) return fail(H3A_EINVAL, "%s: NULL weight or index", fn);
    const int64_t tsize = table_dtype == H3A_DTYPE_F32 ? 4 : 2;
    bool v = cols % 8 == 0 && cols <= h3a::modulate_max_vector_cols() && aligned16(weight);
    for (int i = 0; i < n_tables; ++i) {
        if (rows > 0 && !tables[i]) return fail(H3A_EINVAL, "%s: NULL modulation table", fn);
        if (table_strides[i] < cols) return fail(H3A_EINVAL, "%s: table row stride %lld < cols", fn, (long long)table_strides[i]);
        v = v && aligned16(tables[i]) && (table_strides[i] * tsize) % 16 == 0;
    }
    p.weight = weight;
    p.w_f32 = w_dtype == H3A_DTYPE_F32;
    p.table_f32 = table_dtype == H3A_DTYPE_F32;
    p.index = index;
    p.index_i64 = index_dtype == H3A_DTYPE_I64;
    p.n_index = n_index;
    p.table_rows = table_rows;
    p.rows = rows;
    p.cols = (int32_t)cols;
    p.eps = eps;
    *vec = v;
    return H3A_OK;
}

// A bf16 activation matrix: row stride >= cols; vector path needs 16-byte rows.
int check_rows(const char* fn, const char* name, const void* ptr, int64_t stride, int64_t rows, int64_t cols, bool* vec) {
    if (rows > 0 && !ptr) return fail(H3A_EINVAL, "%s: NULL %s", fn, name);
    if (stride < cols) return fail(H3A_EINVAL, "%s: %s row stride %lld < cols %lld", fn, name, (long long)stride, (long long)cols);
    *vec = *vec && aligned16(ptr) && stride % 8 == 0;
    return H3A_OK;
}

}  // namespace

extern "C" {

const char* h3a_last_error(void) { return g_err; }

int h3a_abi_version(void) { return H3A_ABI_VERSION; }

int h3a_clock_sample(uint64_t* out, void* stream) {
    g_err[0] = '\0';
    if (out == nullptr) return fail(H3A_EINVAL, "h3a_clock_sample: out is NULL");
    if (((uintptr_t)out & 7u) != 0) return fail(H3A_EINVAL, "h3a_clock_sample: out must be 8-byte aligned");
    const hipError_t e = h3a::launch_clock_sample(out, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_clock_sample: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int h3a_attn_fwd(const h3a_attn_args* a, void* stream) {
    g_err[0] = '\0';
    h3a::AttnParams p{};
    bool empty = false;
    const int rc = prepare_attn(a, p, &empty);
    if (rc != H3A_OK || empty) return rc;
    const AttnWorkspace w = attn_workspace(a, p, true);
    if (w.total > 0 && a->workspace != nullptr && a->workspace_bytes >= w.total && ((uintptr_t)a->workspace & 255u) == 0) {
        if (w.plan.split_n != 0) apply_plan(p, w.plan, a->workspace);
        if (w.persist) {
            p.persist_queue = (int*)a->workspace;
            p.persist_blocks = w.cus;
        }
        if (w.ub_tiles > 0) {
            const int64_t pieces = (int64_t)h3a::attn_fwd_tail_pieces() * w.cus;
            p.ws_o = (uint16_t*)a->workspace;
            p.ws_lse = (float*)(p.ws_o + pieces * h3a::attn_fwd_block_m() * 128);
            int32_t* words = (int32_t*)((char*)a->workspace + w.plan_offset);
            p.vplan = p.vplan_w = words;
            p.vlist = p.vlist_w = words + h3a::kPlanWords;
            p.vpieces = p.vpieces_w = p.vlist_w + w.ub_tiles;
            p.vmerge = p.vmerge_w = p.vpieces_w + 2 * pieces;
            p.vscratch = p.vmerge_w + 2 * w.cus;
            p.ub_tiles = w.ub_tiles;
            p.plan_cus = w.cus;
        }
        if (w.vt_rs != 0) {
            p.vt = (char*)a->workspace + w.vt_offset;
            p.vt_rs = (int32_t)w.vt_rs;
            p.vt_sh = 128 * (w.vt_rs / 2);
            p.vt_sb = a->heads * p.vt_sh;
        }
    }
    hipError_t e = h3a::launch_attn_fwd(p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_attn_fwd: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int h3a_attn_fwd_noalloc(const h3a_attn_args* a, void* stream) {
    g_err[0] = '\0';
    h3a::AttnParams p{};
    bool empty = false;
    const int rc = prepare_attn(a, p, &empty);
    if (rc != H3A_OK || empty) return rc;
    void* scratch = nullptr;
    hipError_t e = h3a::attn_static_scratch(&scratch);
    if (e != hipSuccess)
        return fail(H3A_ELAUNCH, "h3a_attn_fwd_noalloc: device scratch lookup failed: %s", hipGetErrorString(e));
    // The plan is fitted to the scratch (fewer key-range pieces, or none), so
    // this only rejects a plan that could not be fitted. No allocation, no
    // memset: the tail's counter is zeroed by a kernel of the launch.
    const h3a::SplitPlan plan = attn_plan(a, p, h3a::kStaticScratchBytes);
    if (plan.workspace_bytes > h3a::kStaticScratchBytes)
        return fail(H3A_EINVAL, "h3a_attn_fwd_noalloc: the launch needs %lld bytes of scratch, the static scratch holds %lld",
                    (long long)plan.workspace_bytes, (long long)h3a::kStaticScratchBytes);
    if (plan.split_n != 0) apply_plan(p, plan, scratch);
    // Packed short segments: the persistent launch, its tile counter in the
    // scratch's first 256 bytes (no split plan uses the scratch then; its
    // zeroing kernel is part of the launch). The planned list's partial
    // results would not fit, so varied lengths take this launch too.
    if (plan.split_n == 0 && a->cu_seqlens_q != nullptr && a->max_seqlen_q <= h3a::attn_fwd_persist_max_rows()) {
        const int cus = device_cus();
        if (cus > 0) {
            p.persist_queue = (int*)scratch;
            p.persist_blocks = cus;
        }
    }
    e = h3a::launch_attn_fwd(p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_attn_fwd_noalloc: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int64_t h3a_attn_fwd_workspace_size(const h3a_attn_args* a) {
    g_err[0] = '\0';
    h3a::AttnParams p{};
    bool empty = false;
    const int rc = prepare_attn(a, p, &empty);
    if (rc != H3A_OK) return rc;
    return empty ? 0 : attn_workspace(a, p, true).total;
}

int h3a_qknorm_rope(const h3a_qknorm_rope_args* a, void* stream) {
    g_err[0] = '\0';
    if (a == nullptr) return fail(H3A_EINVAL, "h3a_qknorm_rope: args is NULL");
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "h3a_qknorm_rope: abi_version %d, library is %d", a->abi_version, H3A_ABI_VERSION);
    const int64_t D = a->head_dim, R = a->rotary_dim;
    if (R > D || R % 2 != 0 || R < 0)
        return fail(H3A_EINVAL,
                    "fused qknorm+rope requires an even rotary dimension no wider than the head, got rotary_dim=%lld, "
                    "head_dim=%lld",
                    (long long)R, (long long)D);
    if (D <= 0 || D % 8 != 0 || D > 512)
        return fail(H3A_EUNSUPPORTED, "h3a_qknorm_rope: head_dim must be a multiple of 8 in [8, 512], got %lld", (long long)D);
    if (a->batch < 0 || a->seqlen < 0 || a->heads <= 0) return fail(H3A_EINVAL, "h3a_qknorm_rope: bad extents");
    if (a->w_dtype != H3A_DTYPE_BF16 && a->w_dtype != H3A_DTYPE_F32)
        return fail(H3A_EINVAL, "h3a_qknorm_rope: unknown weight dtype %d", a->w_dtype);
    if (a->batch == 0 || a->seqlen == 0) return H3A_OK;
    if (!a->xq || !a->yq || !a->wq) return fail(H3A_EINVAL, "h3a_qknorm_rope: NULL q pointer");
    const int n = a->xk ? 2 : 1;
    if (n == 2 && (!a->yk || !a->wk)) return fail(H3A_EINVAL, "h3a_qknorm_rope: xk given without yk/wk");
    if (R > 0 && (!a->cos || !a->sin)) return fail(H3A_EINVAL, "h3a_qknorm_rope: NULL cos/sin table");
    if (R > 0 && a->table_stride < R) return fail(H3A_EINVAL, "h3a_qknorm_rope: table_stride < rotary_dim");
    if (R > 0 && (!aligned4(a->cos) || !aligned4(a->sin)))
        return fail(H3A_EINVAL, "h3a_qknorm_rope: cos/sin must be 4-byte aligned");
    h3a::QkNormRopeParams p{};
    const void* xs[2] = {a->xq, a->xk};
    void* ys[2] = {a->yq, a->yk};
    const void* ws[2] = {a->wq, a->wk};
    const int64_t* xst[2] = {a->xq_stride, a->xk_stride};
    const int64_t* yst[2] = {a->yq_stride, a->yk_stride};
    const float eps[2] = {a->eps_q, a->eps_k};
    for (int i = 0; i < n; ++i) {
        if (!aligned16(xs[i]) || !aligned16(ys[i]) || !aligned16(ws[i]))
            return fail(H3A_EINVAL, "h3a_qknorm_rope: tensors must be 16-byte aligned");
        for (int d = 0; d < 3; ++d)
            if (xst[i][d] % 8 != 0 || yst[i][d] % 8 != 0 || xst[i][d] < 0 || yst[i][d] < 0)
                return fail(H3A_EINVAL, "h3a_qknorm_rope: strides must be non-negative multiples of 8 elements");
        p.x[i] = xs[i]; p.y[i] = ys[i]; p.w[i] = ws[i]; p.eps[i] = eps[i];
        p.x_sb[i] = xst[i][0]; p.x_ss[i] = xst[i][1]; p.x_sh[i] = xst[i][2];
        p.y_sb[i] = yst[i][0]; p.y_ss[i] = yst[i][1]; p.y_sh[i] = yst[i][2];
    }
    if (n == 1) {  // second slot mirrors the first; never selected when n_tensors == 1
        p.x[1] = p.x[0]; p.y[1] = p.y[0]; p.w[1] = p.w[0]; p.eps[1] = p.eps[0];
        p.x_sb[1] = p.x_sb[0]; p.x_ss[1] = p.x_ss[0]; p.x_sh[1] = p.x_sh[0];
        p.y_sb[1] = p.y_sb[0]; p.y_ss[1] = p.y_ss[0]; p.y_sh[1] = p.y_sh[0];
    }
    p.cos = a->cos; p.sin = a->sin; p.table_stride = a->table_stride;
    p.seqlen = (int32_t)a->seqlen; p.heads = (int32_t)a->heads; p.n_tensors = n;
    p.head_dim = (int32_t)D; p.rotary_dim = (int32_t)R; p.w_f32 = a->w_dtype == H3A_DTYPE_F32;
    if ((__int128)a->batch * a->seqlen * n * a->heads >= ((int64_t)1 << 31) || a->batch > 65535)
        return fail(H3A_EUNSUPPORTED, "h3a_qknorm_rope: batch %lld x seqlen %lld x %d x heads %lld rows (limits 2^31, batch 65535)",
                    (long long)a->batch, (long long)a->seqlen, n, (long long)a->heads);
    p.rows = a->batch * a->seqlen * n * a->heads;
    p.div_heads = h3a::make_fast_div((uint32_t)a->heads);
    p.div_tensors = h3a::make_fast_div((uint32_t)n);
    p.div_seqlen = h3a::make_fast_div((uint32_t)a->seqlen);
    p.div_hpg = p.div_heads;  // ungrouped output heads
    hipError_t e = h3a::launch_qknorm_rope(p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_qknorm_rope: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int h3a_pack_qkv(const h3a_pack_qkv_args* a, void* stream) {
    g_err[0] = '\0';
    if (a == nullptr) return fail(H3A_EINVAL, "h3a_pack_qkv: args is NULL");
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "h3a_pack_qkv: abi_version %d, library is %d", a->abi_version, H3A_ABI_VERSION);
    const int64_t es = a->elem_bytes;
    if (es != 1 && es != 2 && es != 4 && es != 8)
        return fail(H3A_EINVAL, "h3a_pack_qkv: elem_bytes must be 1, 2, 4 or 8, got %lld", (long long)es);
    if (a->rows < 0 || a->heads <= 0 || a->head_dim <= 0 || a->world <= 0)
        return fail(H3A_EINVAL, "h3a_pack_qkv: bad extents (rows=%lld heads=%lld head_dim=%lld world=%lld)",
                    (long long)a->rows, (long long)a->heads, (long long)a->head_dim, (long long)a->world);
    if (a->heads % a->world != 0)
        return fail(H3A_EINVAL, "heads (%lld) must divide Ulysses degree (%lld)", (long long)a->heads,
                    (long long)a->world);
    if (a->rows == 0) return H3A_OK;
    if (!a->q || !a->k || !a->v || !a->out) return fail(H3A_EINVAL, "h3a_pack_qkv: NULL tensor pointer");
    const int64_t* st[3] = {a->q_stride, a->k_stride, a->v_stride};
    const void* src[3] = {a->q, a->k, a->v};
    if ((__int128)a->rows * a->heads >= ((int64_t)1 << 31) || a->head_dim >= ((int64_t)1 << 30) / es)
        return fail(H3A_EUNSUPPORTED,
                    "h3a_pack_qkv: rows=%lld heads=%lld head_dim=%lld: (row, head) units and their bytes must stay "
                    "under 2^31 and 2^30",
                    (long long)a->rows, (long long)a->heads, (long long)a->head_dim);
    const int64_t row_bytes = a->head_dim * es;
    h3a::PackQkvParams p{};
    bool vec = row_bytes % 16 == 0 && row_bytes <= 4096 && aligned16(a->out);
    for (int i = 0; i < 3; ++i) {
        if (st[i][0] < 0 || st[i][1] < 0) return fail(H3A_EINVAL, "h3a_pack_qkv: strides must be non-negative");
        p.src[i] = src[i];
        p.s_row[i] = st[i][0] * es;
        p.s_head[i] = st[i][1] * es;
        vec = vec && aligned16(src[i]) && p.s_row[i] % 16 == 0 && p.s_head[i] % 16 == 0;
    }
    p.out = a->out;
    p.rows = a->rows;
    p.row_bytes = (int32_t)row_bytes;
    p.units = (uint32_t)(a->rows * a->heads);
    p.div_heads = h3a::make_fast_div((uint32_t)a->heads);
    p.div_hl = h3a::make_fast_div((uint32_t)(a->heads / a->world));
    hipError_t e = h3a::launch_pack_qkv(p, vec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_pack_qkv: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int h3a_merge_heads(const h3a_merge_heads_args* a, void* stream) {
    g_err[0] = '\0';
    if (a == nullptr) return fail(H3A_EINVAL, "h3a_merge_heads: args is NULL");
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "h3a_merge_heads: abi_version %d, library is %d", a->abi_version, H3A_ABI_VERSION);
    const int64_t es = a->elem_bytes;
    if (es != 1 && es != 2 && es != 4 && es != 8)
        return fail(H3A_EINVAL, "h3a_merge_heads: elem_bytes must be 1, 2, 4 or 8, got %lld", (long long)es);
    if (a->world <= 0 || a->rows < 0 || a->inner < 0)
        return fail(H3A_EINVAL, "h3a_merge_heads: bad extents (world=%lld rows=%lld inner=%lld)", (long long)a->world,
                    (long long)a->rows, (long long)a->inner);
    if (a->x_stride[0] < 0 || a->x_stride[1] < 0) return fail(H3A_EINVAL, "h3a_merge_heads: strides must be non-negative");
    if (a->rows == 0 || a->inner == 0) return H3A_OK;
    if (!a->x || !a->out) return fail(H3A_EINVAL, "h3a_merge_heads: NULL tensor pointer");
    if (a->world >= ((int64_t)1 << 31)) return fail(H3A_EUNSUPPORTED, "h3a_merge_heads: world too large");
    h3a::MergeHeadsParams p{};
    p.x = a->x;
    p.out = a->out;
    p.s_world = a->x_stride[0] * es;
    p.s_row = a->x_stride[1] * es;
    p.rows = a->rows;
    p.inner_bytes = a->inner * es;
    const int64_t vectors = a->rows * a->world * (p.inner_bytes / 16);
    const bool vec = p.inner_bytes % 16 == 0 && aligned16(a->x) && aligned16(a->out) && p.s_world % 16 == 0 &&
                     p.s_row % 16 == 0 && vectors < ((int64_t)1 << 31);
    if (vec) {
        p.vectors = (uint32_t)vectors;
        p.div_inner = h3a::make_fast_div((uint32_t)(p.inner_bytes / 16));
    }
    p.div_world = h3a::make_fast_div((uint32_t)a->world);
    hipError_t e = h3a::launch_merge_heads(p, vec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_merge_heads: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int h3a_qknorm_rope_pack(const h3a_qknorm_rope_pack_args* a, void* stream) {
    g_err[0] = '\0';
    if (a == nullptr) return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: args is NULL");
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: abi_version %d, library is %d", a->abi_version, H3A_ABI_VERSION);
    const int64_t D = a->head_dim, R = a->rotary_dim;
    if (R > D || R % 2 != 0 || R < 0)
        return fail(H3A_EINVAL,
                    "fused qknorm+rope requires an even rotary dimension no wider than the head, got rotary_dim=%lld, "
                    "head_dim=%lld",
                    (long long)R, (long long)D);
    if (D <= 0 || D % 8 != 0 || D > 512)
        return fail(H3A_EUNSUPPORTED, "h3a_qknorm_rope_pack: head_dim must be a multiple of 8 in [8, 512], got %lld",
                    (long long)D);
    if (a->rows < 0 || a->heads <= 0 || a->world <= 0)
        return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: bad extents");
    if (a->heads % a->world != 0)
        return fail(H3A_EINVAL, "heads (%lld) must divide Ulysses degree (%lld)", (long long)a->heads,
                    (long long)a->world);
    if (a->w_dtype != H3A_DTYPE_BF16 && a->w_dtype != H3A_DTYPE_F32)
        return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: unknown weight dtype %d", a->w_dtype);
    if (a->rows == 0) return H3A_OK;
    if (!a->q || !a->k || !a->v || !a->out || !a->wq || !a->wk)
        return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: NULL tensor pointer");
    if (R > 0 && (!a->cos || !a->sin)) return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: NULL cos/sin table");
    if (R > 0 && a->table_stride < R) return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: table_stride < rotary_dim");
    if (R > 0 && (!aligned4(a->cos) || !aligned4(a->sin)))
        return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: cos/sin must be 4-byte aligned");
    const void* ptrs[6] = {a->q, a->k, a->v, a->out, a->wq, a->wk};
    for (const void* q : ptrs)
        if (!aligned16(q)) return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: tensors must be 16-byte aligned");
    const int64_t* st[3] = {a->q_stride, a->k_stride, a->v_stride};
    for (int i = 0; i < 3; ++i)
        for (int d = 0; d < 2; ++d)
            if (st[i][d] < 0 || st[i][d] % 8 != 0)
                return fail(H3A_EINVAL, "h3a_qknorm_rope_pack: strides must be non-negative multiples of 8 elements");
    if ((__int128)a->rows * 2 * a->heads >= ((int64_t)1 << 31))
        return fail(H3A_EUNSUPPORTED, "h3a_qknorm_rope_pack: %lld rows (limit 2^31 / (2 * heads))", (long long)a->rows);
    const int64_t hl = a->heads / a->world;
    const int64_t slot = 3 * D;         // one head's q|k|v in the packed buffer
    const int64_t row_stride = hl * slot;  // one row of one destination
    const int64_t group_stride = a->rows * row_stride;  // one destination
    uint16_t* out = (uint16_t*)a->out;
    h3a::QkNormRopeParams p{};
    p.x[0] = a->q; p.x[1] = a->k;
    p.y[0] = out; p.y[1] = out + D;
    p.w[0] = a->wq; p.w[1] = a->wk;
    p.eps[0] = a->eps_q; p.eps[1] = a->eps_k;
    for (int i = 0; i < 2; ++i) {
        p.x_sb[i] = 0; p.x_ss[i] = st[i][0]; p.x_sh[i] = st[i][1];
        p.y_sb[i] = 0; p.y_ss[i] = row_stride; p.y_sh[i] = slot; p.y_sg[i] = group_stride;
    }
    p.xc = a->v; p.yc = out + 2 * D;
    p.xc_sb = 0; p.xc_ss = a->v_stride[0]; p.xc_sh = a->v_stride[1];
    p.yc_sb = 0; p.yc_ss = row_stride; p.yc_sh = slot; p.yc_sg = group_stride;
    p.cos = a->cos; p.sin = a->sin; p.table_stride = a->table_stride;
    p.seqlen = (int32_t)a->rows; p.heads = (int32_t)a->heads; p.n_tensors = 2;
    p.head_dim = (int32_t)D; p.rotary_dim = (int32_t)R; p.w_f32 = a->w_dtype == H3A_DTYPE_F32;
    p.rows = a->rows * 2 * a->heads;
    p.div_heads = h3a::make_fast_div((uint32_t)a->heads);
    p.div_tensors = h3a::make_fast_div(2u);
    p.div_seqlen = h3a::make_fast_div((uint32_t)a->rows);
    p.div_hpg = h3a::make_fast_div((uint32_t)hl);
    // Rotary widths that are not a multiple of 16, or tables without 16-byte
    // rows, take the generic kernel (one row per lane group, element-wise
    // partner and table reads) in the same output layout.
    hipError_t e = h3a::launch_qknorm_rope(p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "h3a_qknorm_rope_pack: launch failed: %s", hipGetErrorString(e));
    return H3A_OK;
}

int h3a_rmsnorm_modulate(const h3a_rmsnorm_modulate_args* a, void* stream) {
    g_err[0] = '\0';
    const char* fn = "h3a_rmsnorm_modulate";
    if (a == nullptr) return fail(H3A_EINVAL, "%s: args is NULL", fn);
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "%s: abi_version %d, library is %d", fn, a->abi_version, H3A_ABI_VERSION);
    h3a::ModulateParams p{};
    bool vec = false;
    const void* tables[2] = {a->scale, a->shift};
    const int64_t strides[2] = {a->scale_stride, a->shift_stride};
    int rc = prepare_modulate(fn, a->weight, a->w_dtype, tables, strides, 2, a->table_dtype, a->table_rows, a->index,
                              a->index_dtype, a->n_index, a->rows, a->cols, a->eps, p, &vec);
    if (rc != H3A_OK) return rc;
    if ((rc = check_rows(fn, "x", a->x, a->x_stride, a->rows, a->cols, &vec)) != H3A_OK) return rc;
    if ((rc = check_rows(fn, "out", a->out, a->out_stride, a->rows, a->cols, &vec)) != H3A_OK) return rc;
    if (a->rows == 0) return H3A_OK;
    p.x = a->x; p.out = a->out; p.scale = a->scale; p.shift = a->shift;
    p.x_stride = a->x_stride; p.out_stride = a->out_stride;
    p.scale_stride = a->scale_stride; p.shift_stride = a->shift_stride;
    hipError_t e = h3a::launch_modulate(p, vec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return H3A_OK;
}

int h3a_residual_gate_rmsnorm_modulate(const h3a_residual_gate_rmsnorm_modulate_args* a, void* stream) {
    g_err[0] = '\0';
    const char* fn = "h3a_residual_gate_rmsnorm_modulate";
    if (a == nullptr) return fail(H3A_EINVAL, "%s: args is NULL", fn);
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "%s: abi_version %d, library is %d", fn, a->abi_version, H3A_ABI_VERSION);
    h3a::ModulateParams p{};
    bool vec = false;
    const void* tables[3] = {a->gate, a->scale, a->shift};
    const int64_t strides[3] = {a->gate_stride, a->scale_stride, a->shift_stride};
    int rc = prepare_modulate(fn, a->weight, a->w_dtype, tables, strides, 3, a->table_dtype, a->table_rows, a->index,
                              a->index_dtype, a->n_index, a->rows, a->cols, a->eps, p, &vec);
    if (rc != H3A_OK) return rc;
    if ((rc = check_rows(fn, "residual", a->residual, a->residual_stride, a->rows, a->cols, &vec)) != H3A_OK) return rc;
    if ((rc = check_rows(fn, "branch", a->branch, a->branch_stride, a->rows, a->cols, &vec)) != H3A_OK) return rc;
    if ((rc = check_rows(fn, "hidden_out", a->hidden_out, a->hidden_stride, a->rows, a->cols, &vec)) != H3A_OK) return rc;
    if ((rc = check_rows(fn, "normed_out", a->normed_out, a->normed_stride, a->rows, a->cols, &vec)) != H3A_OK) return rc;
    if (a->rows == 0) return H3A_OK;
    p.x = a->branch; p.residual = a->residual; p.out = a->normed_out; p.hidden = a->hidden_out;
    p.gate = a->gate; p.scale = a->scale; p.shift = a->shift;
    p.x_stride = a->branch_stride; p.residual_stride = a->residual_stride;
    p.out_stride = a->normed_stride; p.hidden_stride = a->hidden_stride;
    p.gate_stride = a->gate_stride; p.scale_stride = a->scale_stride; p.shift_stride = a->shift_stride;
    hipError_t e = h3a::launch_modulate(p, vec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return H3A_OK;
}

int h3a_swiglu(const h3a_swiglu_args* a, void* stream) {
    g_err[0] = '\0';
    const char* fn = "h3a_swiglu";
    if (a == nullptr) return fail(H3A_EINVAL, "%s: args is NULL", fn);
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "%s: abi_version %d, library is %d", fn, a->abi_version, H3A_ABI_VERSION);
    if (a->rows < 0 || a->cols < 0) return fail(H3A_EINVAL, "%s: bad extents", fn);
    if (a->x_stride < 2 * a->cols || a->out_stride < a->cols)
        return fail(H3A_EINVAL, "%s: row strides must cover the row (x: 2*cols, out: cols)", fn);
    if (a->rows == 0 || a->cols == 0) return H3A_OK;
    if (!a->x || !a->out) return fail(H3A_EINVAL, "%s: NULL tensor pointer", fn);
    h3a::SwigluParams p{a->x, a->out, a->x_stride, a->out_stride, a->rows, a->cols};
    const bool vec = a->cols % 8 == 0 && aligned16(a->x) && aligned16(a->out) && a->x_stride % 8 == 0 &&
                     a->out_stride % 8 == 0;
    hipError_t e = h3a::launch_swiglu(p, vec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return H3A_OK;
}

int h3a_attn_merge(const h3a_attn_merge_args* a, void* stream) {
    g_err[0] = '\0';
    const char* fn = "h3a_attn_merge";
    if (a == nullptr) return fail(H3A_EINVAL, "%s: args is NULL", fn);
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "%s: abi_version %d, library is %d", fn, a->abi_version, H3A_ABI_VERSION);
    if (a->n_parts < 1 || a->n_parts > H3A_MERGE_MAX_PARTS)
        return fail(H3A_EINVAL, "%s: n_parts must be in [1, %d], got %d", fn, H3A_MERGE_MAX_PARTS, a->n_parts);
    if (a->batch < 0 || a->heads <= 0 || a->seqlen < 0 || a->head_dim <= 0)
        return fail(H3A_EINVAL, "%s: bad extents", fn);
    if (a->head_dim % 8 != 0 || a->head_dim > 512)
        return fail(H3A_EUNSUPPORTED, "%s: head_dim must be a multiple of 8 in [8, 512], got %lld", fn, (long long)a->head_dim);
    const bool pf = a->part_dtype == H3A_DTYPE_F32, of = a->out_dtype == H3A_DTYPE_F32;
    if ((!pf && a->part_dtype != H3A_DTYPE_BF16) || (!of && a->out_dtype != H3A_DTYPE_BF16))
        return fail(H3A_EINVAL, "%s: part and out dtypes must be bf16 or fp32", fn);
    if (a->batch == 0 || a->seqlen == 0) return H3A_OK;
    if ((__int128)a->batch * a->seqlen * a->heads >= ((int64_t)1 << 40) || a->heads >= ((int64_t)1 << 31) ||
        a->seqlen >= ((int64_t)1 << 31))
        return fail(H3A_EUNSUPPORTED, "%s: too many rows (batch x seqlen x heads under 2^40, heads and seqlen under 2^31)",
                    fn);
    if (!a->o) return fail(H3A_EINVAL, "%s: NULL output", fn);
    const int64_t psz = pf ? 4 : 2, osz = of ? 4 : 2;
    h3a::AttnMergeParams p{};
    for (int i = 0; i < a->n_parts; ++i) {
        if (!a->o_parts[i] || !a->lse_parts[i]) return fail(H3A_EINVAL, "%s: NULL part %d", fn, i);
        if (!aligned16(a->o_parts[i])) return fail(H3A_EINVAL, "%s: part %d must be 16-byte aligned", fn, i);
        if (!aligned4(a->lse_parts[i])) return fail(H3A_EINVAL, "%s: LSE of part %d must be 4-byte aligned", fn, i);
        p.o_parts[i] = a->o_parts[i];
        p.lse_parts[i] = a->lse_parts[i];
    }
    for (int d = 0; d < 3; ++d)
        if (a->part_o_stride[d] < 0 || a->o_stride[d] < 0 || (a->part_o_stride[d] * psz) % 16 != 0 ||
            (a->o_stride[d] * osz) % 16 != 0)
            return fail(H3A_EINVAL, "%s: output strides must be non-negative and keep rows 16-byte aligned", fn);
    if (!aligned16(a->o)) return fail(H3A_EINVAL, "%s: out must be 16-byte aligned", fn);
    if (a->lse != nullptr && !aligned4(a->lse)) return fail(H3A_EINVAL, "%s: lse must be 4-byte aligned", fn);
    if (a->part_lse_stride[0] < 0 || a->part_lse_stride[1] < 0 || a->lse_stride[0] < 0 || a->lse_stride[1] < 0)
        return fail(H3A_EINVAL, "%s: LSE strides must be non-negative", fn);
    p.o = a->o;
    p.lse = a->lse;
    p.po_sb = a->part_o_stride[0]; p.po_ss = a->part_o_stride[1]; p.po_sh = a->part_o_stride[2];
    p.pl_sb = a->part_lse_stride[0]; p.pl_sh = a->part_lse_stride[1];
    p.o_sb = a->o_stride[0]; p.o_ss = a->o_stride[1]; p.o_sh = a->o_stride[2];
    p.l_sb = a->lse_stride[0]; p.l_sh = a->lse_stride[1];
    p.n_parts = a->n_parts;
    p.heads = (int32_t)a->heads; p.seqlen = (int32_t)a->seqlen; p.head_dim = (int32_t)a->head_dim;
    p.rows = a->batch * a->seqlen * a->heads;
    p.part_f32 = pf; p.out_f32 = of;
    hipError_t e = h3a::launch_attn_merge(p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return H3A_OK;
}

int h3a_proj_gemm(const h3a_proj_args* a, void* stream) {
    g_err[0] = '\0';
    const char* fn = "h3a_proj_gemm";
    if (a == nullptr) return fail(H3A_EINVAL, "%s: args is NULL", fn);
    if (a->abi_version != H3A_ABI_VERSION)
        return fail(H3A_EINVAL, "%s: abi_version %d, library is %d", fn, a->abi_version, H3A_ABI_VERSION);
    if (a->head_dim != 128) return fail(H3A_EUNSUPPORTED, "%s: head_dim must be 128, got %lld", fn, (long long)a->head_dim);
    if (a->num_sections < 1 || a->num_sections > H3A_PROJ_MAX_SECTIONS)
        return fail(H3A_EINVAL, "%s: num_sections must be in [1, %d], got %d", fn, H3A_PROJ_MAX_SECTIONS, a->num_sections);
    if (a->m < 0 || a->k <= 0) return fail(H3A_EINVAL, "%s: bad extents (m=%lld k=%lld)", fn, (long long)a->m, (long long)a->k);
    const int64_t step = h3a::proj_gemm_k_multiple();
    if (a->k % step != 0)
        return fail(H3A_EUNSUPPORTED, "%s: k must be a multiple of %lld, got %lld", fn, (long long)step, (long long)a->k);
    const int64_t R = a->rotary_dim;
    bool any_norm = false;
    for (int i = 0; i < a->num_sections; ++i) any_norm |= a->sections[i].mode == H3A_PROJ_QKNORM_ROPE;
    if (any_norm && (R < 0 || R > 128 || R % 2 != 0))
        return fail(H3A_EINVAL,
                    "fused qknorm+rope requires an even rotary dimension no wider than the head, got rotary_dim=%lld, "
                    "head_dim=128",
                    (long long)R);
    if (!a->x || !aligned16(a->x)) return fail(H3A_EINVAL, "%s: x must be a 16-byte aligned device pointer", fn);
    if (a->x_stride < a->k || a->x_stride % 8 != 0)
        return fail(H3A_EINVAL, "%s: x_stride must be a multiple of 8 elements and at least k", fn);
    const int64_t tile = h3a::proj_gemm_tile();
    // Every buffer resource spans one tile of rows from its base.
    const int64_t span_limit = ((int64_t)1 << 32) - 1;
    // rows * stride_elems * 2 + tail_bytes, checked without overflowing int64
    auto spans = [&](int64_t rows, int64_t stride, int64_t tail) {
        return stride <= (span_limit - tail) / 2 / rows;
    };
    if (a->k > span_limit / 2 || !spans(tile - 1, a->x_stride, a->k * 2))
        return fail(H3A_EUNSUPPORTED, "%s: x_stride too large", fn);
    if (a->m >= ((int64_t)1 << 31)) return fail(H3A_EUNSUPPORTED, "%s: m too large", fn);
    h3a::ProjGemmParams p{};
    p.x = a->x;
    p.x_rs = a->x_stride * 2;
    p.m = (int32_t)a->m;
    p.k = (int32_t)a->k;
    p.n_sections = a->num_sections;
    int64_t n_tiles = 0;
    for (int i = 0; i < a->num_sections; ++i) {
        const h3a_proj_section& s = a->sections[i];
        if (s.mode != H3A_PROJ_PLAIN && s.mode != H3A_PROJ_QKNORM_ROPE)
            return fail(H3A_EINVAL, "%s: section %d: unknown mode %d", fn, i, s.mode);
        if (s.n <= 0 || s.n % 128 != 0 || s.n >= ((int64_t)1 << 30))
            return fail(H3A_EUNSUPPORTED, "%s: section %d: n must be a positive multiple of 128, got %lld", fn, i,
                        (long long)s.n);
        if (!s.weight || !s.y || !aligned16(s.weight) || !aligned16(s.y))
            return fail(H3A_EINVAL, "%s: section %d: weight and y must be 16-byte aligned device pointers", fn, i);
        if (s.weight_stride < a->k || s.weight_stride % 8 != 0 || s.y_stride < s.n || s.y_stride % 8 != 0)
            return fail(H3A_EINVAL, "%s: section %d: strides must be multiples of 8 elements covering the row", fn, i);
        if (!spans(tile - 1, s.weight_stride, a->k * 2))
            return fail(H3A_EUNSUPPORTED, "%s: section %d: weight_stride too large", fn, i);
        // A wave's output resource spans half a tile of token rows.
        if (!spans(tile / 2 - 1, s.y_stride, 256))
            return fail(H3A_EUNSUPPORTED, "%s: section %d: y_stride too large", fn, i);
        if (s.bias && ((uintptr_t)s.bias & 7u) != 0)
            return fail(H3A_EINVAL, "%s: section %d: bias must be 8-byte aligned", fn, i);
        if (s.mode == H3A_PROJ_QKNORM_ROPE) {
            if (!s.norm_weight || ((uintptr_t)s.norm_weight & 7u) != 0)
                return fail(H3A_EINVAL, "%s: section %d: norm_weight must be an 8-byte aligned device pointer", fn, i);
            if (!(s.eps >= 0.f) || !isfinite(s.eps)) return fail(H3A_EINVAL, "%s: section %d: bad eps", fn, i);
        }
        h3a::ProjSection& d = p.sec[i];
        d.w = s.weight;
        d.bias = s.bias;
        d.norm_w = s.norm_weight;
        d.y = s.y;
        d.w_rs = s.weight_stride * 2;
        d.y_rs = s.y_stride * 2;
        d.n = (int32_t)s.n;
        d.tiles = (int32_t)((s.n + tile - 1) / tile);
        d.mode = s.mode;
        d.eps = s.eps;
        n_tiles += d.tiles;
    }
    if (any_norm && R > 0) {
        if (!a->cos || !a->sin) return fail(H3A_EINVAL, "%s: NULL cos/sin table", fn);
        if (a->seqlen <= 0 || a->seqlen >= ((int64_t)1 << 31)) return fail(H3A_EINVAL, "%s: seqlen must be in [1, 2^31)", fn);
        if (a->table_stride < R) return fail(H3A_EINVAL, "%s: table_stride < rotary_dim", fn);
        if (a->table_stride > span_limit / 4 / a->seqlen)
            return fail(H3A_EUNSUPPORTED, "%s: cos/sin tables must span less than 2^32 bytes", fn);
        if (!aligned4(a->cos) || !aligned4(a->sin)) return fail(H3A_EINVAL, "%s: cos/sin must be 4-byte aligned", fn);
        p.cos = a->cos;
        p.sin = a->sin;
        p.table_stride = a->table_stride;
        p.rotary_dim = (int32_t)R;
        p.seqlen = (int32_t)a->seqlen;
        // The in-lane epilogue (partners in the same lane, only the first
        // half of the tables read) needs R a multiple of 32, the caller's
        // word that the tables are in the rotate-half form, and 16-byte
        // table rows; anything else reads the tables at every column.
        const bool in_lane = R % 32 == 0 && a->rotate_half_tables == 1 && aligned16(a->cos) && aligned16(a->sin) &&
                             a->table_stride % 4 == 0;
        p.rope_full_tables = in_lane ? 0 : 1;
    } else {
        p.rotary_dim = 0;
        p.seqlen = 1;
    }
    // Sections without RoPE store their rows straight from registers, unless
    // the launch has RoPE sections or writes rows of 16 KiB or more: then
    // they stage them in LDS and write whole 256-byte pieces past the
    // caches, like the RoPE sections (the 40-head q/k/v launch 0.6% faster,
    // three plain 5,120-wide sections 3.8%; one such section measured 0.8%
    // slower staged).
    int64_t out_row_bytes = 0;
    for (int i = 0; i < a->num_sections; ++i) out_row_bytes += a->sections[i].n * 2;
    p.stage_plain = (any_norm && R > 0) || out_row_bytes >= 16384 ? 1 : 0;
    if (a->m == 0) return H3A_OK;
    p.m_tiles = (int32_t)((a->m + tile - 1) / tile);
    p.n_tiles = (int32_t)n_tiles;
    if ((int64_t)p.m_tiles * n_tiles >= ((int64_t)1 << 31)) return fail(H3A_EUNSUPPORTED, "%s: grid too large", fn);
    hipError_t e = h3a::launch_proj_gemm(p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(H3A_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return H3A_OK;
}

}  // extern "C"
