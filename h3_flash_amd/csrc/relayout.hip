// Bit-exact relayouts on either side of the packed-Ulysses exchange (gfx950).
//
// pack_qkv: q, k, v of shape (rows, heads, D) -> out (world, rows, heads/world,
// 3*D), destination-major: the slice out[d] holds the heads d*hl .. d*hl+hl-1
// (hl = heads/world) of every row, with q, k and v of one head side by side.
// Same movement as the reference Triton kernel _pack_qkv_kernel
// (src/h3_flash/runtime/parallel/relayout.py:11-49):
//   out[dest][row][lh][i*D + d] = X_i[row][dest*hl + lh][d],  X = (q, k, v).
//
// merge_heads: x (world, rows, inner) -> out (rows, world, inner), the
// source-rank / row transpose of relayout.py:52-67,133-159:
//   out[row][src][t] = x[src][row][t].
//
// Both are pure data movement, HBM-bound: every byte is read once and written
// once. The vector paths move 16 bytes per lane with non-temporal accesses;
// the byte paths serve shapes whose rows are not 16-byte multiples.
#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kThreads = 256;

// One group of L lanes per (row, head) unit; lane j moves bytes [16j, 16j+16)
// of the head's row in each of the three tensors.
// Threads per workgroup of the vector pack: 128 measured 3.5% faster than
// 256 on a Ulysses rank's shard (at least one lane group per workgroup).
constexpr int pack_threads(int lanes) { return lanes > 128 ? lanes : 128; }

template <int L>
__global__ __launch_bounds__(pack_threads(L)) void pack_qkv_kernel(PackQkvParams p) {
    const uint32_t unit = blockIdx.x * (uint32_t)(pack_threads(L) / L) + threadIdx.x / L;
    const int j = threadIdx.x % L;
    if (unit >= p.units || j * 16 >= p.row_bytes) return;
    const uint32_t row = fdiv(unit, p.div_heads);
    const uint32_t h = unit - row * p.div_heads.d;
    const uint32_t dest = fdiv(h, p.div_hl);
    const uint32_t lh = h - dest * p.div_hl.d;
    char* o = (char*)p.out + (((int64_t)dest * p.rows + row) * p.div_hl.d + lh) * 3 * p.row_bytes + j * 16;
    i32x4 v[3];
#pragma unroll
    for (int i = 0; i < 3; ++i)
        v[i] = __builtin_nontemporal_load(
            (const i32x4*)((const char*)p.src[i] + (int64_t)row * p.s_row[i] + (int64_t)h * p.s_head[i] + j * 16));
#pragma unroll
    for (int i = 0; i < 3; ++i) __builtin_nontemporal_store(v[i], (i32x4*)(o + i * p.row_bytes));
}

// Byte path: one thread per byte of the packed output.
__global__ __launch_bounds__(kThreads) void pack_qkv_bytes_kernel(PackQkvParams p) {
    const int64_t total = (int64_t)p.units * 3 * p.row_bytes;
    for (int64_t o = blockIdx.x * (int64_t)kThreads + threadIdx.x; o < total; o += (int64_t)gridDim.x * kThreads) {
        const int64_t slot = o / p.row_bytes;  // (dest, row, lh, i)
        const int byte = (int)(o - slot * p.row_bytes);
        const int i = (int)(slot % 3);
        const int64_t head_slot = slot / 3;  // (dest, row, lh)
        const int64_t lh = head_slot % p.div_hl.d;
        const int64_t row_slot = head_slot / p.div_hl.d;  // (dest, row)
        const int64_t row = row_slot % p.rows;
        const int64_t dest = row_slot / p.rows;
        const int64_t h = dest * p.div_hl.d + lh;
        ((char*)p.out)[o] = ((const char*)p.src[i])[row * p.s_row[i] + h * p.s_head[i] + byte];
    }
}

// Output vector o (16 bytes) -> (row, src, t); reads x[src][row] at vector t.
__global__ __launch_bounds__(kThreads) void merge_heads_kernel(MergeHeadsParams p) {
    const uint32_t o = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
    if (o >= p.vectors) return;
    const uint32_t blk = fdiv(o, p.div_inner);  // (row, src)
    const uint32_t t = o - blk * p.div_inner.d;
    const uint32_t row = fdiv(blk, p.div_world);
    const uint32_t src = blk - row * p.div_world.d;
    const i32x4 v = __builtin_nontemporal_load(
        (const i32x4*)((const char*)p.x + (int64_t)src * p.s_world + (int64_t)row * p.s_row + (int64_t)t * 16));
    __builtin_nontemporal_store(v, (i32x4*)p.out + o);
}

__global__ __launch_bounds__(kThreads) void merge_heads_bytes_kernel(MergeHeadsParams p) {
    const int64_t total = (int64_t)p.rows * p.div_world.d * p.inner_bytes;
    for (int64_t o = blockIdx.x * (int64_t)kThreads + threadIdx.x; o < total; o += (int64_t)gridDim.x * kThreads) {
        const int64_t blk = o / p.inner_bytes;
        const int64_t t = o - blk * p.inner_bytes;
        const int64_t row = blk / p.div_world.d;
        const int64_t src = blk - row * p.div_world.d;
        ((char*)p.out)[o] = ((const char*)p.x)[src * p.s_world + row * p.s_row + t];
    }
}

unsigned byte_grid(int64_t total) {
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    return (unsigned)(blocks < 65536 ? blocks : 65536);
}

}  // namespace

hipError_t launch_pack_qkv(const PackQkvParams& p, bool vec, hipStream_t stream) {
    if (p.units == 0) return hipSuccess;
    if (!vec) {
        hipLaunchKernelGGL(pack_qkv_bytes_kernel, dim3(byte_grid((int64_t)p.units * 3 * p.row_bytes)), dim3(kThreads),
                           0, stream, p);
        return hipGetLastError();
    }
    int lanes = 1;
    while (lanes * 16 < p.row_bytes) lanes <<= 1;
    auto go = [&](auto kernel, int l) {
        const int threads = pack_threads(l), per = threads / l;
        const unsigned blocks = (unsigned)(((int64_t)p.units + per - 1) / per);
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(threads), 0, stream, p);
        return hipGetLastError();
    };
    switch (lanes) {
        case 1: return go(pack_qkv_kernel<1>, 1);
        case 2: return go(pack_qkv_kernel<2>, 2);
        case 4: return go(pack_qkv_kernel<4>, 4);
        case 8: return go(pack_qkv_kernel<8>, 8);
        case 16: return go(pack_qkv_kernel<16>, 16);
        case 32: return go(pack_qkv_kernel<32>, 32);
        case 64: return go(pack_qkv_kernel<64>, 64);
        case 128: return go(pack_qkv_kernel<128>, 128);
        case 256: return go(pack_qkv_kernel<256>, 256);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_merge_heads(const MergeHeadsParams& p, bool vec, hipStream_t stream) {
    if (vec) {
        if (p.vectors == 0) return hipSuccess;
        hipLaunchKernelGGL(merge_heads_kernel, dim3((p.vectors + kThreads - 1) / kThreads), dim3(kThreads), 0, stream,
                           p);
    } else {
        const int64_t total = (int64_t)p.rows * p.div_world.d * p.inner_bytes;
        if (total == 0) return hipSuccess;
        hipLaunchKernelGGL(merge_heads_bytes_kernel, dim3(byte_grid(total)), dim3(kThreads), 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace h3a
