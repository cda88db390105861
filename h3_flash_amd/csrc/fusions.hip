// Row-wise fusions of the MiniMax H3 DiT block around attention (gfx950).
//
// Arithmetic follows the reference Triton kernels
// (src/h3_flash/runtime/kernels/fusions.py), in fp32 with one rounding on
// store:
//   rmsnorm_modulate (:69-96)
//       n   = x * rsqrt(sum(x^2) / C + eps)
//       out = n * w * (1 + scale[t]) + shift[t]
//   residual_gate_rmsnorm_modulate (:23-67)
//       h      = residual + gate[t] * branch          -> hidden_out
//       n      = h * rsqrt(sum(h^2) / C + eps) * w    (h in fp32, unrounded)
//       normed = n * (1 + scale[t]) + shift[t]        -> normed_out
//   swiglu (:98-123)
//       out = value * (gate * sigmoid(gate)),  value = x[:, :C], gate = x[:, C:]
// with t = index[row % n_index] the modulation-table row of a token.
//
// Layout and roofline: each row kernel keeps its row in VGPRs (one 256-thread
// workgroup per row, 16 bytes per lane per vector), so x (and residual,
// branch) are read from HBM once and the outputs written once; weight and the
// small modulation tables are re-read by every row and served from L2. All
// kernels are HBM-bound. Indices outside the table are clamped to it (the
// reference reads out of bounds there).
#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kThreads = 256;  // one row per workgroup in the norm kernels
constexpr int kWaves = kThreads / 64;
constexpr int kSwigluThreads = 128;  // measured 4.5% faster than 256 for swiglu

__device__ __forceinline__ void unpack8(i32x4 raw, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = (uint32_t)raw[i];
        f[2 * i] = __uint_as_float(w << 16);
        f[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
    }
}

__device__ __forceinline__ i32x4 pack8(const float* f) {
    i32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (int)pack_bf16x2(f[2 * i], f[2 * i + 1]);
    return r;
}

__device__ __forceinline__ float load1(const void* base, int64_t idx, bool f32) {
    return f32 ? ((const float*)base)[idx] : bf16_to_f32(((const uint16_t*)base)[idx]);
}

__device__ __forceinline__ int64_t table_row(const ModulateParams& p, int64_t row) {
    const int64_t i = row % p.n_index;
    int64_t t = p.index_i64 ? ((const int64_t*)p.index)[i] : (int64_t)((const int32_t*)p.index)[i];
    t = t < 0 ? 0 : t;
    return t >= p.table_rows ? p.table_rows - 1 : t;
}

// Sum of v over the workgroup (fixed order: lanes, then waves in order).
__device__ __forceinline__ float block_sum(float v, float* lds) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += lds[w];
    return s;
}

// Eight consecutive bf16 (16 bytes) or fp32 (32 bytes) values as loaded,
// unpacked only when used, so that many loads can be in flight at once.
template <bool kF32>
struct Raw8 {
    i32x4 a;
    i32x4 b;  // second half of fp32 values; unused for bf16
};

template <bool kF32>
__device__ __forceinline__ Raw8<kF32> fetch8(const void* base, int64_t idx) {
    Raw8<kF32> r;
    if constexpr (kF32) {
        r.a = *(const i32x4*)((const float*)base + idx);
        r.b = *(const i32x4*)((const float*)base + idx + 4);
    } else {
        r.a = *(const i32x4*)((const uint16_t*)base + idx);
    }
    return r;
}

template <bool kF32>
__device__ __forceinline__ void unpack_raw8(const Raw8<kF32>& r, float* out) {
    if constexpr (kF32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[i] = __int_as_float(r.a[i]);
            out[4 + i] = __int_as_float(r.b[i]);
        }
    } else {
        unpack8(r.a, out);
    }
}

// Vector path: C % 8 == 0, every row and table row 16-byte aligned.
// NV = vectors of 8 per thread, the fewest with NV * 8 * kThreads >= C, so a
// thread's vectors 0 .. NV-2 always lie inside the row and only the last may
// not. That one is loaded from the row's last vector instead and dropped.
// Every load of a phase is then issued without a branch between loads, and
// all of them are in flight together (a load behind a bounds branch is
// waited for before the next one is issued). Table dtypes are template
// arguments for the same reason.
template <int NV, bool kResidual, bool kTabF32, bool kWF32>
__global__ __launch_bounds__(kThreads) void modulate_kernel(ModulateParams p) {
    __shared__ float red[kWaves];
    const int64_t row = blockIdx.x;
    const int C = p.cols;
    const int64_t t = table_row(p, row);
    int col[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) col[k] = (threadIdx.x + k * kThreads) * 8;
    const bool last = col[NV - 1] < C;  // the last vector lies inside the row
    if (!last) col[NV - 1] = C - 8;

    const uint16_t* xr = (const uint16_t*)p.x + row * p.x_stride;
    i32x4 rx[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) rx[k] = __builtin_nontemporal_load((const i32x4*)(xr + col[k]));
    float h[NV][8];
    float ss = 0.f;
    if constexpr (kResidual) {
        const uint16_t* rr = (const uint16_t*)p.residual + row * p.residual_stride;
        i32x4 rres[NV];
        Raw8<kTabF32> g[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) rres[k] = __builtin_nontemporal_load((const i32x4*)(rr + col[k]));
#pragma unroll
        for (int k = 0; k < NV; ++k) g[k] = fetch8<kTabF32>(p.gate, t * p.gate_stride + col[k]);
        uint16_t* hr = (uint16_t*)p.hidden + row * p.hidden_stride;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float r[8], b[8], gv[8];
            unpack8(rres[k], r);
            unpack8(rx[k], b);
            unpack_raw8<kTabF32>(g[k], gv);
#pragma unroll
            for (int e = 0; e < 8; ++e) h[k][e] = r[e] + gv[e] * b[e];
            if (k < NV - 1 || last) {
                __builtin_nontemporal_store(pack8(h[k]), (i32x4*)(hr + col[k]));
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += h[k][e] * h[k][e];
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            unpack8(rx[k], h[k]);
            if (k < NV - 1 || last)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += h[k][e] * h[k][e];
        }
    }
    // Weight and table rows are issued before the reduction, so their latency
    // overlaps it.
    Raw8<kWF32> w[NV];
    Raw8<kTabF32> sc[NV], sh[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        w[k] = fetch8<kWF32>(p.weight, col[k]);
        sc[k] = fetch8<kTabF32>(p.scale, t * p.scale_stride + col[k]);
        sh[k] = fetch8<kTabF32>(p.shift, t * p.shift_stride + col[k]);
    }
    const float r = rsqrtf(block_sum(ss, red) / (float)C + p.eps);
    uint16_t* orow = (uint16_t*)p.out + row * p.out_stride;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (k == NV - 1 && !last) break;
        float wv[8], scv[8], shv[8], o[8];
        unpack_raw8<kWF32>(w[k], wv);
        unpack_raw8<kTabF32>(sc[k], scv);
        unpack_raw8<kTabF32>(sh[k], shv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = h[k][e] * r * wv[e] * (1.0f + scv[e]) + shv[e];
        __builtin_nontemporal_store(pack8(o), (i32x4*)(orow + col[k]));
    }
}

// Wave path (C % 8 == 0, C <= 64 * 8 * kRowVecMax, 16-byte aligned rows):
// one wave per row, four rows per workgroup, which share the weight row
// through LDS (one barrier). Each wave issues its row's loads (x, or
// residual and branch, and the gate row) and then every scale and shift
// vector it will need, all before the first wait, and holds its outputs
// until the end: on gfx9 one counter covers loads and stores, so a store
// issued ahead of a load would make that load's wait also wait for the
// store. The row index, and so the row bases and the modulation-table row,
// are wave-uniform (scalar registers; lanes add 32-bit offsets). Measured
// against the one-row-per-workgroup kernel above on 49,920 x 5,120 rows:
// 5.4 -> 6.0 TB/s (rmsnorm_modulate) and 5.3 -> 6.1 TB/s (residual
// variant); at 6,240 rows within 2%. Used for bf16 tables up to 11 vectors
// per lane (C <= 5,632), where it keeps two waves per SIMD; the block kernel
// takes the rest.
constexpr int kRowVecMax = 11;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <bool kTabF32>
struct RowTabs {
    Raw8<kTabF32> sc, sh;
};

// Eight values at byte offset `off` (of the bf16 column) of a row that starts
// at `base`: a uniform base and a 32-bit lane offset, one address register.
template <bool kF32>
__device__ __forceinline__ Raw8<kF32> fetch8o(const char* base, uint32_t off) {
    Raw8<kF32> r;
    if constexpr (kF32) {
        r.a = *(const i32x4*)(base + 2 * off);
        r.b = *(const i32x4*)(base + 2 * off + 16);
    } else {
        r.a = *(const i32x4*)(base + off);
    }
    return r;
}

template <int NV, bool kResidual, bool kTabF32, bool kWF32>
__global__ __launch_bounds__(kThreads) void modulate_row_kernel(ModulateParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t row_id = (int64_t)blockIdx.x * kWaves + wave;  // uniform: row bases and t in scalar registers
    const bool live = row_id < p.rows;
    const int64_t row = live ? row_id : p.rows - 1;  // a wave past the rows loads the last one, stores nothing
    const int C = p.cols;
    // Vectors 0 .. NV-2 of a lane lie inside the row (NV = ceil(C / 512));
    // the last one, where it does not, is loaded from the row's last vector
    // and dropped. off[k]: byte offset of vector k in a bf16 row.
    uint32_t off[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) off[k] = (uint32_t)(lane + 64 * k) * 16u;
    const bool last = (int)(off[NV - 1] / 2) < C;
    if (!last) off[NV - 1] = (uint32_t)(C - 8) * 2u;

    const char* xr = (const char*)p.x + row * p.x_stride * 2;
    i32x4 rx[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) rx[k] = __builtin_nontemporal_load((const i32x4*)(xr + off[k]));
    i32x4 rres[kResidual ? NV : 1];
    if constexpr (kResidual) {
        const char* rr = (const char*)p.residual + row * p.residual_stride * 2;
#pragma unroll
        for (int k = 0; k < NV; ++k) rres[k] = __builtin_nontemporal_load((const i32x4*)(rr + off[k]));
    }
    const int64_t t = table_row(p, row);
    const int tb_sz = kTabF32 ? 4 : 2;
    const char* const wrow = (const char*)p.weight;
    const char* const scrow = (const char*)p.scale + t * p.scale_stride * tb_sz;
    const char* const shrow = (const char*)p.shift + t * p.shift_stride * tb_sz;
    // The weight row, shared by the workgroup's four rows, goes through LDS:
    // vector i (columns 8i .. 8i+7, the last clamped into the row) at wl[i].
    constexpr int kWv = NV * 64, kWl = kWF32 ? 2 : 1;
    __shared__ i32x4 wl[kWv * kWl];
    {
        constexpr int kIt = (kWv + kThreads - 1) / kThreads;
        Raw8<kWF32> wv[kIt];
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int i = min((int)threadIdx.x + it * kThreads, kWv - 1);
            wv[it] = fetch8o<kWF32>(wrow, (uint32_t)min(i * 8, C - 8) * 2u);
        }
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int i = min((int)threadIdx.x + it * kThreads, kWv - 1);
            wl[i * kWl] = wv[it].a;
            if constexpr (kWF32) wl[i * kWl + 1] = wv[it].b;
        }
    }
    auto tabs = [&](int k) __attribute__((always_inline)) {
        return RowTabs<kTabF32>{fetch8o<kTabF32>(scrow, off[k]), fetch8o<kTabF32>(shrow, off[k])};
    };
    float ss = 0.f;
    float h[kResidual ? NV : 1][8];
    if constexpr (kResidual) {
        const char* const grow = (const char*)p.gate + t * p.gate_stride * tb_sz;
        Raw8<kTabF32> g[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) g[k] = fetch8o<kTabF32>(grow, off[k]);
        char* const hr = (char*)p.hidden + row * p.hidden_stride * 2;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float r[8], b[8], gv[8];
            unpack_raw8<kTabF32>(g[k], gv);
            unpack8(rres[k], r);
            unpack8(rx[k], b);
#pragma unroll
            for (int e = 0; e < 8; ++e) h[k][e] = r[e] + gv[e] * b[e];
            if (live && (k < NV - 1 || last)) {
                __builtin_nontemporal_store(pack8(h[k]), (i32x4*)(hr + off[k]));
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += h[k][e] * h[k][e];
            }
        }
    }
    RowTabs<kTabF32> tb[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) tb[k] = tabs(k);
    if constexpr (!kResidual) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float v[8];
            unpack8(rx[k], v);
            if (k < NV - 1 || last)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
        }
        // Unpack x again below rather than keep the fp32 values of the sum
        // live through it (twice the registers of the raw vectors).
#pragma unroll
        for (int k = 0; k < NV; ++k) asm volatile("" : "+v"(rx[k]));
    }
    const float r = rsqrtf(wave_sum(ss) / (float)C + p.eps);
    __syncthreads();  // the weight row is in LDS
    if (!live) return;
    i32x4 ov[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float v[8], wv[8], scv[8], shv[8], o[8];
        if constexpr (kResidual) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = h[k][e];
        } else {
            unpack8(rx[k], v);
        }
        {
            Raw8<kWF32> w;
            w.a = wl[(lane + 64 * k) * kWl];
            if constexpr (kWF32) w.b = wl[(lane + 64 * k) * kWl + 1];
            unpack_raw8<kWF32>(w, wv);
        }
        unpack_raw8<kTabF32>(tb[k].sc, scv);
        unpack_raw8<kTabF32>(tb[k].sh, shv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = v[e] * r * wv[e] * (1.0f + scv[e]) + shv[e];
        ov[k] = pack8(o);
    }
    char* const orow = (char*)p.out + row * p.out_stride * 2;
#pragma unroll
    for (int k = 0; k < NV; ++k)
        if (k < NV - 1 || last) __builtin_nontemporal_store(ov[k], (i32x4*)(orow + off[k]));
}

// Element path (any C, any alignment): two passes over the row, the second
// re-reading x (or the unrounded residual + gate * branch) from cache.
template <bool kResidual>
__global__ __launch_bounds__(kThreads) void modulate_elem_kernel(ModulateParams p) {
    __shared__ float red[kWaves];
    const int64_t row = blockIdx.x;
    const int C = p.cols;
    const int64_t t = table_row(p, row);
    auto value = [&](int c) {
        if constexpr (kResidual) {
            const float r = bf16_to_f32(((const uint16_t*)p.residual)[row * p.residual_stride + c]);
            const float b = bf16_to_f32(((const uint16_t*)p.x)[row * p.x_stride + c]);
            return r + load1(p.gate, t * p.gate_stride + c, p.table_f32) * b;
        } else {
            return bf16_to_f32(((const uint16_t*)p.x)[row * p.x_stride + c]);
        }
    };
    float ss = 0.f;
    for (int c = threadIdx.x; c < C; c += kThreads) {
        const float h = value(c);
        ss += h * h;
        if constexpr (kResidual) {
            const uint32_t bits = pack_bf16x2(h, 0.f);
            ((uint16_t*)p.hidden)[row * p.hidden_stride + c] = (uint16_t)(bits & 0xffffu);
        }
    }
    const float r = rsqrtf(block_sum(ss, red) / (float)C + p.eps);
    for (int c = threadIdx.x; c < C; c += kThreads) {
        const float o = value(c) * r * load1(p.weight, c, p.w_f32) * (1.0f + load1(p.scale, t * p.scale_stride + c, p.table_f32)) +
                        load1(p.shift, t * p.shift_stride + c, p.table_f32);
        const uint32_t bits = pack_bf16x2(o, 0.f);
        ((uint16_t*)p.out)[row * p.out_stride + c] = (uint16_t)(bits & 0xffffu);
    }
}

__device__ __forceinline__ float silu_mul(float v, float g) { return v * (g * (1.0f / (1.0f + __expf(-g)))); }

// out[r, c] = x[r, c] * silu(x[r, C + c]); vector o covers 8 columns.
__global__ __launch_bounds__(kSwigluThreads) void swiglu_kernel(SwigluParams p) {
    const int64_t per_row = p.cols / 8;
    const int64_t total = p.rows * per_row;
    for (int64_t o = blockIdx.x * (int64_t)kSwigluThreads + threadIdx.x; o < total; o += (int64_t)gridDim.x * kSwigluThreads) {
        const int64_t row = o / per_row;
        const int64_t c = (o - row * per_row) * 8;
        const uint16_t* x = (const uint16_t*)p.x + row * p.x_stride + c;
        float v[8], g[8], out[8];
        unpack8(__builtin_nontemporal_load((const i32x4*)x), v);
        unpack8(__builtin_nontemporal_load((const i32x4*)(x + p.cols)), g);
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = silu_mul(v[e], g[e]);
        __builtin_nontemporal_store(pack8(out), (i32x4*)((uint16_t*)p.out + row * p.out_stride + c));
    }
}

__global__ __launch_bounds__(kSwigluThreads) void swiglu_elem_kernel(SwigluParams p) {
    const int64_t total = p.rows * p.cols;
    for (int64_t o = blockIdx.x * (int64_t)kSwigluThreads + threadIdx.x; o < total; o += (int64_t)gridDim.x * kSwigluThreads) {
        const int64_t row = o / p.cols;
        const int64_t c = o - row * p.cols;
        const uint16_t* x = (const uint16_t*)p.x + row * p.x_stride;
        const uint32_t bits = pack_bf16x2(silu_mul(bf16_to_f32(x[c]), bf16_to_f32(x[p.cols + c])), 0.f);
        ((uint16_t*)p.out)[row * p.out_stride + c] = (uint16_t)(bits & 0xffffu);
    }
}

unsigned stride_grid(int64_t work) {
    const int64_t blocks = (work + kSwigluThreads - 1) / kSwigluThreads;
    return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

template <bool kResidual, bool kTabF32, bool kWF32>
void launch_modulate_vec(const ModulateParams& p, int nv, hipStream_t stream) {
    const int nw = (int)((p.cols + 511) / 512);  // vectors per lane with one wave per row
    if constexpr (!kTabF32) {
        if (nw <= kRowVecMax) {
            const dim3 grid((unsigned)((p.rows + kWaves - 1) / kWaves)), block(kThreads);
            switch (nw) {
#define H3A_NW(n)                                                                                                     \
    case n:                                                                                                           \
        hipLaunchKernelGGL((modulate_row_kernel<n, kResidual, kTabF32, kWF32>), grid, block, 0, stream, p);         \
        break;
                H3A_NW(1) H3A_NW(2) H3A_NW(3) H3A_NW(4) H3A_NW(5) H3A_NW(6) H3A_NW(7) H3A_NW(8)
                H3A_NW(9) H3A_NW(10) H3A_NW(11)
#undef H3A_NW
            }
            return;
        }
    }
    const dim3 grid((unsigned)p.rows), block(kThreads);
    switch (nv) {
#define H3A_NV(n)                                                                                                     \
    case n:                                                                                                           \
        hipLaunchKernelGGL((modulate_kernel<n, kResidual, kTabF32, kWF32>), grid, block, 0, stream, p);             \
        break;
        H3A_NV(1) H3A_NV(2) H3A_NV(3) H3A_NV(4) H3A_NV(5) H3A_NV(6) H3A_NV(7) H3A_NV(8)
#undef H3A_NV
    }
}

template <bool kResidual>
hipError_t launch_modulate_t(const ModulateParams& p, bool vec, hipStream_t stream) {
    const int nv = (int)((p.cols + 8 * kThreads - 1) / (8 * kThreads));
    if (!vec || nv < 1 || nv > 8) {
        hipLaunchKernelGGL((modulate_elem_kernel<kResidual>), dim3((unsigned)p.rows), dim3(kThreads), 0, stream, p);
    } else if (p.table_f32) {
        if (p.w_f32)
            launch_modulate_vec<kResidual, true, true>(p, nv, stream);
        else
            launch_modulate_vec<kResidual, true, false>(p, nv, stream);
    } else {
        if (p.w_f32)
            launch_modulate_vec<kResidual, false, true>(p, nv, stream);
        else
            launch_modulate_vec<kResidual, false, false>(p, nv, stream);
    }
    return hipGetLastError();
}

}  // namespace

int modulate_max_vector_cols() { return 8 * 8 * kThreads; }

hipError_t launch_modulate(const ModulateParams& p, bool vec, hipStream_t stream) {
    if (p.rows == 0 || p.cols == 0) return hipSuccess;
    return p.residual != nullptr ? launch_modulate_t<true>(p, vec, stream) : launch_modulate_t<false>(p, vec, stream);
}

hipError_t launch_swiglu(const SwigluParams& p, bool vec, hipStream_t stream) {
    if (p.rows == 0 || p.cols == 0) return hipSuccess;
    if (vec)
        hipLaunchKernelGGL(swiglu_kernel, dim3(stride_grid(p.rows * (p.cols / 8))), dim3(kSwigluThreads), 0, stream, p);
    else
        hipLaunchKernelGGL(swiglu_elem_kernel, dim3(stride_grid(p.rows * p.cols)), dim3(kSwigluThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace h3a
