// Merge of partial attention results over disjoint key ranges (gfx950): the
// combine step of ring / context-parallel attention, applied to the (out,
// lse) pairs a forward op returns for each key chunk:
//   lse = m + log(sum_p exp(lse_p - m)),  m = max_p lse_p
//   out = sum_p exp(lse_p - lse) * out_p
// in fp32. Parts whose LSE is -inf (no keys) weigh nothing; a row with no
// keys in any part gets out = 0 and lse = -inf.
//
// One lane group of D/8 lanes per (batch, seq, head) row, 8 columns per lane.
// Every part's row is read before the row is written, so the output may
// alias one of the parts (in-place online merging). HBM-bound: per row it
// reads n_parts * D elements and writes D.
#include <math.h>

#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kThreads = 128;  // 128 measured 3% faster than 256 or 512

// kPF32: partial outputs are fp32 (else bf16); kMaxP >= n_parts sizes the
// registers that hold the loaded rows (4, 8 or 16, so a small merge keeps a
// high occupancy). Every LSE and every part row of the call is loaded in one
// unrolled sequence before any is used: no load waits behind another's
// value, and the rows do not wait for the LSEs. The sequence ends on a
// wave-uniform branch at n_parts; with 16 slots it ends only at a multiple of
// 4 (the compiler keeps it unrolled then), and a slot past n_parts reloads
// the last part, dropped by a select.
template <int L, bool kPF32, int kMaxP>
__global__ __launch_bounds__(kThreads) void attn_merge_parts_kernel(AttnMergeParams p) {
    // Workgroup i runs on XCD i % 8. For one or two bf16 parts, each XCD takes
    // one contiguous range of rows, so a 64-byte line of the (B, H, S) LSEs,
    // shared by 16 tokens whose rows span about 10 workgroups, is fetched
    // into one XCD's L2 rather than several (2 parts at B=1 S=49,920 H=5:
    // 33 -> 30 us). A bijection on [0, gridDim.x). With more parts, or fp32
    // parts, dispatch order measured as fast or faster.
    uint32_t blk = blockIdx.x;
    if (!kPF32 && p.n_parts <= 2) {
        const uint32_t nb = gridDim.x, per = nb / 8, rem = nb % 8, x = blk % 8;
        blk = x * per + min(x, rem) + blk / 8;
    }
    const int64_t row = (int64_t)blk * (kThreads / L) + threadIdx.x / L;
    const int j = threadIdx.x % L;
    if (row >= p.rows || j * 8 >= p.head_dim) return;
    const int64_t h = row % p.heads;
    const int64_t bs = row / p.heads;
    const int64_t s = bs % p.seqlen;
    const int64_t b = bs / p.seqlen;
    const int64_t lse_off = b * p.pl_sb + h * p.pl_sh + s;
    const int64_t o_off = b * p.po_sb + s * p.po_ss + h * p.po_sh + j * 8;
    const int n = p.n_parts;
    constexpr int kStep = kMaxP > 8 ? 4 : 1;  // slots between early exits
    float lq[kMaxP];
    i32x4 ra[kMaxP], rb[kPF32 ? kMaxP : 1];
#pragma unroll
    for (int q = 0; q < kMaxP; ++q) {
        if (q % kStep == 0 && q >= n) break;
        const int qc = q < n ? q : n - 1;
        lq[q] = p.lse_parts[qc][lse_off];
        if constexpr (kPF32) {
            const float* src = (const float*)p.o_parts[qc] + o_off;
            ra[q] = *(const i32x4*)src;
            rb[q] = *(const i32x4*)(src + 4);
        } else {
            ra[q] = *(const i32x4*)((const uint16_t*)p.o_parts[qc] + o_off);
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMaxP; ++q) {
        if (q % kStep == 0 && q >= n) break;
        if (q < n) m = fmaxf(m, lq[q]);
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
#pragma unroll
    for (int q = 0; q < kMaxP; ++q) {
        if (q % kStep == 0 && q >= n) break;
        // A part with no keys (lse = -inf), or a reloaded slot, weighs
        // nothing, and its row (possibly garbage) is replaced by zeros.
        const bool use = q < n && lq[q] != -INFINITY;
        const float w = use ? __expf(lq[q] - m) : 0.f;
        float v[8];
        if constexpr (kPF32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = __int_as_float(ra[q][e]);
                v[4 + e] = __int_as_float(rb[q][e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = __uint_as_float(((uint32_t)ra[q][e]) << 16);
                v[2 * e + 1] = __uint_as_float(((uint32_t)ra[q][e]) & 0xffff0000u);
            }
        }
        wsum += w;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(w, use ? v[e] : 0.f, acc[e]);
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    const int64_t out = b * p.o_sb + s * p.o_ss + h * p.o_sh + j * 8;
    if (p.out_f32) {
        float* o = (float*)p.o + out;
        *(f32x4*)o = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        *(f32x4*)(o + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    } else {
        i32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (int)pack_bf16x2(acc[2 * i] * inv, acc[2 * i + 1] * inv);
        *(i32x4*)((uint16_t*)p.o + out) = w;
    }
    if (p.lse != nullptr && j == 0) p.lse[b * p.l_sb + h * p.l_sh + s] = wsum > 0.f ? m + __logf(wsum) : -INFINITY;
}

template <int L>
hipError_t launch_l(const AttnMergeParams& p, hipStream_t stream) {
    const int64_t per = kThreads / L;
    const dim3 grid((unsigned)((p.rows + per - 1) / per));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, p);
        return hipGetLastError();
    };
    const bool f = p.part_f32 != 0;
    if (p.n_parts <= 4) return f ? go(attn_merge_parts_kernel<L, true, 4>) : go(attn_merge_parts_kernel<L, false, 4>);
    if (p.n_parts <= 8) return f ? go(attn_merge_parts_kernel<L, true, 8>) : go(attn_merge_parts_kernel<L, false, 8>);
    return f ? go(attn_merge_parts_kernel<L, true, 16>) : go(attn_merge_parts_kernel<L, false, 16>);
}

}  // namespace

hipError_t launch_attn_merge(const AttnMergeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    static_assert(kMergeMaxParts == 16, "part-count buckets are 4, 8 and 16");
    int lanes = 1;
    while (lanes * 8 < p.head_dim) lanes <<= 1;
    switch (lanes) {
        case 1: return launch_l<1>(p, stream);
        case 2: return launch_l<2>(p, stream);
        case 4: return launch_l<4>(p, stream);
        case 8: return launch_l<8>(p, stream);
        case 16: return launch_l<16>(p, stream);
        case 32: return launch_l<32>(p, stream);
        case 64: return launch_l<64>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace h3a
