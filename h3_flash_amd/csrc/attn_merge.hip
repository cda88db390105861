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
constexpr int kBatch = 4;  // part rows in flight per lane (4 measured faster than 8 or 16)

template <int L>
__global__ __launch_bounds__(kThreads) void attn_merge_parts_kernel(AttnMergeParams p) {
    const int64_t row = (int64_t)blockIdx.x * (kThreads / L) + threadIdx.x / L;
    const int j = threadIdx.x % L;
    if (row >= p.rows || j * 8 >= p.head_dim) return;
    const int64_t h = row % p.heads;
    const int64_t bs = row / p.heads;
    const int64_t s = bs % p.seqlen;
    const int64_t b = bs / p.seqlen;
    const int64_t lse_off = b * p.pl_sb + h * p.pl_sh + s;
    const int64_t o_off = b * p.po_sb + s * p.po_ss + h * p.po_sh + j * 8;
    // Every LSE first, then the part rows in batches of kBatch whose loads are
    // all issued before any is used (a load whose value is used in its own
    // conditional block is waited for before the next load issues).
    float lq[kMergeMaxParts];
#pragma unroll
    for (int q = 0; q < kMergeMaxParts; ++q) lq[q] = q < p.n_parts ? p.lse_parts[q][lse_off] : -INFINITY;
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMergeMaxParts; ++q) m = fmaxf(m, lq[q]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    const bool f32 = p.part_f32 != 0;
    if (m != -INFINITY) {
#pragma unroll
        for (int q0 = 0; q0 < kMergeMaxParts; q0 += kBatch) {
            if (q0 >= p.n_parts) break;
            i32x4 ra[kBatch], rb[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const int q = q0 + i;
                if (q < p.n_parts) {
                    if (f32) {
                        ra[i] = *(const i32x4*)((const float*)p.o_parts[q] + o_off);
                        rb[i] = *(const i32x4*)((const float*)p.o_parts[q] + o_off + 4);
                    } else {
                        ra[i] = *(const i32x4*)((const uint16_t*)p.o_parts[q] + o_off);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const int q = q0 + i;
                if (q >= p.n_parts) break;
                if (lq[q] == -INFINITY) continue;
                const float w = __expf(lq[q] - m);
                float v[8];
                if (f32) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = __int_as_float(ra[i][e]);
                        v[4 + e] = __int_as_float(rb[i][e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] = __uint_as_float(((uint32_t)ra[i][e]) << 16);
                        v[2 * e + 1] = __uint_as_float(((uint32_t)ra[i][e]) & 0xffff0000u);
                    }
                }
                wsum += w;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] += w * v[e];
            }
        }
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

}  // namespace

hipError_t launch_attn_merge(const AttnMergeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    int lanes = 1;
    while (lanes * 8 < p.head_dim) lanes <<= 1;
    auto go = [&](auto kernel, int l) {
        const int64_t per = kThreads / l;
        hipLaunchKernelGGL(kernel, dim3((unsigned)((p.rows + per - 1) / per)), dim3(kThreads), 0, stream, p);
        return hipGetLastError();
    };
    switch (lanes) {
        case 1: return go(attn_merge_parts_kernel<1>, 1);
        case 2: return go(attn_merge_parts_kernel<2>, 2);
        case 4: return go(attn_merge_parts_kernel<4>, 4);
        case 8: return go(attn_merge_parts_kernel<8>, 8);
        case 16: return go(attn_merge_parts_kernel<16>, 16);
        case 32: return go(attn_merge_parts_kernel<32>, 32);
        case 64: return go(attn_merge_parts_kernel<64>, 64);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace h3a
