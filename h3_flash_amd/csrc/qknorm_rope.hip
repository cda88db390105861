// Fused per-head RMSNorm + rotate-half RoPE for q and k in one launch (gfx950).
//
// Arithmetic per (token s, head h) row follows the reference Triton kernel
// _qknorm_partial_rope_kernel (src/h3_flash/runtime/kernels/fusions.py:126-175):
//   variance = sum(x*x) / D ; r = rsqrt(variance + eps) ; n = (x * r) * w
//   partner  = c + R/2 (c < R/2) or c - R/2 (R/2 <= c < R)
//   y[c]     = n[c]*cos[s,c] + rot[c]*sin[s,c],  rot = -n[partner] / +n[partner]
//   y[c]     = n[c] for c >= R
// all in fp32, rounded once to bf16. The token of a row is its sequence index
// s (fusions.py:141), so one cos/sin row serves every head of q and k.
//
// Layout: a row of D bf16 values is handled by L = D/8 lanes, 16 bytes each.
// Rows are numbered (batch, token, tensor, head) with the head fastest, so the
// 2*H rows of one token are processed by neighbouring lanes and read their
// cos/sin row from HBM once. The kernel is HBM-bound: per token it moves
// 2*H*D*2 bytes in, the same out, and 2*R*4 bytes of tables.
#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void unpack8(i32x4 raw, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = (uint32_t)raw[i];
        f[2 * i] = __uint_as_float(w << 16);
        f[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
    }
}

__device__ __forceinline__ float load_w(const void* w, int idx, bool f32) {
    return f32 ? ((const float*)w)[idx] : bf16_to_f32(((const uint16_t*)w)[idx]);
}

// Eight consecutive weights starting at a multiple of 8 (16/32-byte aligned).
__device__ __forceinline__ void load_w8(const void* w, int col0, bool f32, float* out) {
    if (f32) {
        const f32x4 a = *(const f32x4*)((const float*)w + col0);
        const f32x4 b = *(const f32x4*)((const float*)w + col0 + 4);
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
        unpack8(*(const i32x4*)((const uint16_t*)w + col0), out);
    }
}

// L lanes per row; kFast: R % 16 == 0 and 16-byte aligned tables, so a lane's
// 8 columns are either all rotary or all pass-through, its partner columns are
// the 8 columns of lane (j +- R/16), and cos/sin come in two 16-byte loads.
template <int L, bool kFast>
__global__ __launch_bounds__(kThreads) void qknorm_rope_kernel(QkNormRopeParams p) {
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / L) + tid / L;
    const int j = tid % L;
    const int D = p.head_dim, R = p.rotary_dim, half = R >> 1;
    // Lanes of a row past the end still join the shuffles below.
    const bool row_ok = row < p.rows;
    const int64_t rr = row_ok ? row : 0;
    const int h = (int)(rr % p.heads);
    int64_t t = rr / p.heads;
    const int which = (int)(t % p.n_tensors);
    t /= p.n_tensors;
    const int s = (int)(t % p.seqlen);
    const int64_t b = t / p.seqlen;

    const uint16_t* x = (const uint16_t*)p.x[which] + b * p.x_sb[which] + s * p.x_ss[which] + h * p.x_sh[which];
    uint16_t* y = (uint16_t*)p.y[which] + b * p.y_sb[which] + s * p.y_ss[which] + h * p.y_sh[which];
    const void* w = p.w[which];
    const bool wf = p.w_f32 != 0;

    const int col0 = j * 8;
    const bool active = row_ok && col0 < D;
    float xv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (active) unpack8(*(const i32x4*)(x + col0), xv);

    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += xv[i] * xv[i];
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, L);
    const float r = rsqrtf(ss / (float)D + p.eps[which]);

    float out[8];
    if constexpr (kFast) {
        // Partner chunk lives in lane j +- R/16 of the same row.
        const bool rot = col0 < R;
        const bool first = col0 < half;
        const int src = rot ? (first ? j + half / 8 : j - half / 8) : j;
        uint32_t mine[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)  // re-pack the own chunk (exact: values came from bf16)
            mine[i] = (__float_as_uint(xv[2 * i]) >> 16) | (__float_as_uint(xv[2 * i + 1]) & 0xffff0000u);
        i32x4 praw;
#pragma unroll
        for (int i = 0; i < 4; ++i) praw[i] = __shfl((int)mine[i], src, L);
        float xp[8];
        unpack8(praw, xp);
        float wv[8];
        if (active) load_w8(w, col0, wf, wv);
        if (rot && active) {
            float wp[8];
            load_w8(w, src * 8, wf, wp);
            const float* cp = p.cos + (int64_t)s * p.table_stride + col0;
            const float* sp = p.sin + (int64_t)s * p.table_stride + col0;
            const f32x4 c0 = *(const f32x4*)cp, c1 = *(const f32x4*)(cp + 4);
            const f32x4 s0 = *(const f32x4*)sp, s1 = *(const f32x4*)(sp + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float n = xv[i] * r * wv[i];
                const float pn = xp[i] * r * wp[i];
                const float rt = first ? -pn : pn;
                out[i] = n * cv[i] + rt * sv[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) out[i] = active ? xv[i] * r * wv[i] : 0.f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int col = col0 + i;
            float o = 0.f;
            if (active && col < D) {
                const float n = xv[i] * r * load_w(w, col, wf);
                if (col < R) {
                    const bool first = col < half;
                    const int pc = first ? col + half : col - half;
                    const float pn = bf16_to_f32(x[pc]) * r * load_w(w, pc, wf);
                    const float rt = first ? -pn : pn;
                    const float cv = p.cos[(int64_t)s * p.table_stride + col];
                    const float sv = p.sin[(int64_t)s * p.table_stride + col];
                    o = n * cv + rt * sv;
                } else {
                    o = n;
                }
            }
            out[i] = o;
        }
    }
    if (active) {
        i32x4 packed;
#pragma unroll
        for (int i = 0; i < 4; ++i) packed[i] = (int)pack_bf16x2(out[2 * i], out[2 * i + 1]);
        *(i32x4*)(y + col0) = packed;
    }
}

template <bool kFast>
hipError_t launch_l(const QkNormRopeParams& p, hipStream_t stream) {
    int lanes = 1;
    while (lanes * 8 < p.head_dim) lanes <<= 1;
    const int64_t rows_per_block = kThreads / lanes;
    const unsigned blocks = (unsigned)((p.rows + rows_per_block - 1) / rows_per_block);
    switch (lanes) {
        case 1: hipLaunchKernelGGL((qknorm_rope_kernel<1, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        case 2: hipLaunchKernelGGL((qknorm_rope_kernel<2, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        case 4: hipLaunchKernelGGL((qknorm_rope_kernel<4, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        case 8: hipLaunchKernelGGL((qknorm_rope_kernel<8, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        case 16: hipLaunchKernelGGL((qknorm_rope_kernel<16, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        case 32: hipLaunchKernelGGL((qknorm_rope_kernel<32, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        case 64: hipLaunchKernelGGL((qknorm_rope_kernel<64, kFast>), dim3(blocks), dim3(kThreads), 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_qknorm_rope(const QkNormRopeParams& p, hipStream_t stream) {
    if (p.rows <= 0) return hipSuccess;
    const bool aligned = ((uintptr_t)p.cos % 16 == 0) && ((uintptr_t)p.sin % 16 == 0) && (p.table_stride % 4 == 0);
    const bool fast = (p.rotary_dim % 16 == 0) && aligned;
    return fast ? launch_l<true>(p, stream) : launch_l<false>(p, stream);
}

}  // namespace h3a
