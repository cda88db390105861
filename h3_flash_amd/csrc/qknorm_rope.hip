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
// The kernel is HBM-bound: per token it moves 2*H*D*2 bytes in, the same out,
// and 2*R*4 bytes of tables.
#include "common.h"
#include "kernels.h"

namespace h3a {

FastDiv make_fast_div(uint32_t d) {
    uint32_t s = 0;
    while (s < 32 && ((uint64_t)1 << s) < d) ++s;
    const uint64_t m = (((uint64_t)1 << 32) * (((uint64_t)1 << s) - d)) / d + 1;
    return FastDiv{d, (uint32_t)m, s};
}

namespace {

constexpr int kThreads = 128;  // 128 measured 1-2% faster than 256 (the pack mode and the prologue alike)
// Heads per lane group in the fast path. With a copied third tensor a group
// holds three tensors' rows in flight, and 4 heads (114 VGPRs, 4 waves per
// SIMD) measured 8% faster than 8 (162 VGPRs, 3 waves) on a Ulysses rank's
// shard; 2 heads was slower again. Without a copy, 8 is fastest.
constexpr int kHeadChunk = 8;
constexpr int kHeadChunkCopy = 4;

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

// Element offset of output head h: (h / hpg) * sg + (h % hpg) * sh.
__device__ __forceinline__ int64_t head_ofs(const QkNormRopeParams& p, int h, int64_t sh, int64_t sg) {
    const uint32_t g = fdiv((uint32_t)h, p.div_hpg);
    return (int64_t)g * sg + (int64_t)((uint32_t)h - g * p.div_hpg.d) * sh;
}

struct RowRef {
    const uint16_t* x;
    uint16_t* y;
    uint32_t s, h, b;
    int which;
    bool ok;
};

__device__ __forceinline__ RowRef locate(const QkNormRopeParams& p, uint32_t row) {
    RowRef r;
    r.ok = row < (uint32_t)p.rows;
    const uint32_t rr = r.ok ? row : 0u;
    const uint32_t t = fdiv(rr, p.div_heads);
    r.h = rr - t * p.div_heads.d;
    const uint32_t t2 = fdiv(t, p.div_tensors);
    r.which = (int)(t - t2 * p.div_tensors.d);
    r.b = fdiv(t2, p.div_seqlen);
    r.s = t2 - r.b * p.div_seqlen.d;
    const bool second = r.which != 0;
    r.x = (const uint16_t*)(second ? p.x[1] : p.x[0]) + (int64_t)r.b * (second ? p.x_sb[1] : p.x_sb[0]) +
          (int64_t)r.s * (second ? p.x_ss[1] : p.x_ss[0]) + (int64_t)r.h * (second ? p.x_sh[1] : p.x_sh[0]);
    r.y = (uint16_t*)(second ? p.y[1] : p.y[0]) + (int64_t)r.b * (second ? p.y_sb[1] : p.y_sb[0]) +
          (int64_t)r.s * (second ? p.y_ss[1] : p.y_ss[0]) +
          head_ofs(p, (int)r.h, second ? p.y_sh[1] : p.y_sh[0], second ? p.y_sg[1] : p.y_sg[0]);
    return r;
}

// Fast path: R % 16 == 0 and 16-byte aligned tables, so a lane's 8 columns
// are either all rotary or all pass-through, its partner columns are the 8
// columns of lane (j +- R/16), and cos/sin come in two 16-byte loads.
// One lane group per (token, chunk of kChunk heads): it reads the token's
// cos/sin once and walks its heads tensor by tensor, each tensor's loads
// issued first (with a copied third tensor, all loads of the block first);
// tensor and head are uniform over the block (scalar indexing).
// Splitting heads over blockIdx.y keeps the grid wide for short shards with
// many heads (a Ulysses rank's 6,240 rows x 40 heads). Every byte of x and y
// is touched once: non-temporal accesses.
template <int L, bool kCopy>
__global__ __launch_bounds__(kThreads, kCopy ? 3 : 4) void qknorm_rope_kernel(QkNormRopeParams p) {
    constexpr int kGroups = kThreads / L;
    constexpr int kChunk = kCopy ? kHeadChunkCopy : kHeadChunk;
    const int tid = threadIdx.x;
    const int j = tid % L;
    const int s = (int)blockIdx.x * kGroups + tid / L;  // token
    const int64_t b = blockIdx.z;
    const int D = p.head_dim, R = p.rotary_dim, half = R >> 1;
    const int hb = (int)blockIdx.y * kChunk;  // this block's heads: [hb, H)
    const int H = min(p.heads, hb + kChunk);
    const int col0 = j * 8;
    const bool on = s < p.seqlen && col0 < D;
    const bool rot = col0 < R;
    const bool first = col0 < half;
    const int src = rot ? (first ? j + half / 8 : j - half / 8) : j;
    const bool ror8 = R == 8 * L;  // every lane rotary, partner j ^ (L / 2)
    const bool wf = p.w_f32 != 0;
    const float inv_d = 1.0f / (float)D;
    const bool d_pow2 = (D & (D - 1)) == 0;  // then ss * inv_d == ss / D exactly

    float cv[8], sv[8];
    if (on && rot) {
        const float* cp = p.cos + (int64_t)s * p.table_stride + col0;
        const float* sp = p.sin + (int64_t)s * p.table_stride + col0;
        const f32x4 c0 = *(const f32x4*)cp, c1 = *(const f32x4*)(cp + 4);
        const f32x4 s0 = *(const f32x4*)sp, s1 = *(const f32x4*)(sp + 4);
        cv[0] = c0.x; cv[1] = c0.y; cv[2] = c0.z; cv[3] = c0.w; cv[4] = c1.x; cv[5] = c1.y; cv[6] = c1.z; cv[7] = c1.w;
        sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w; sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
    }

    // Normalise, rotate and store one row chunk (all L lanes of the group join
    // the reductions and the partner shuffle).
    auto row = [&](const i32x4& x, const float* wv, const float* wp, float eps, uint16_t* dst) __attribute__((always_inline)) {
        float xv[8];
        unpack8(x, xv);
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
        if constexpr (L <= 16) {
            ss = group_sum<L>(ss);
        } else {
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, L);
        }
        const float r = rsqrtf((d_pow2 ? ss * inv_d : ss / (float)D) + eps);
        // Partner chunk lives in lane src of the same row; with R = D = 128
        // that is lane j ^ 8 of the 16, a DPP rotation of the row.
        i32x4 praw;
        if (L == 16 && ror8) {
#pragma unroll
            for (int e = 0; e < 4; ++e) praw[e] = dpp<kDppRor8>(x[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) praw[e] = __shfl(x[e], src, L);
        }
        if (!on) return;
        float out[8];
        if (rot) {
            float xp[8];
            unpack8(praw, xp);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float n = xv[e] * r * wv[e];
                const float pn = xp[e] * r * wp[e];
                const float rt = first ? -pn : pn;
                out[e] = n * cv[e] + rt * sv[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) out[e] = xv[e] * r * wv[e];
        }
        i32x4 packed;
#pragma unroll
        for (int e = 0; e < 4; ++e) packed[e] = (int)pack_bf16x2(out[2 * e], out[2 * e + 1]);
        __builtin_nontemporal_store(packed, (i32x4*)dst);
    };
    const int nh = H - hb;  // heads of this block (uniform)
    auto x_at = [&](int which, int i) {
        return (const i32x4*)((const uint16_t*)p.x[which] + b * p.x_sb[which] + (int64_t)s * p.x_ss[which] + col0 +
                              (int64_t)(hb + i) * p.x_sh[which]);
    };
    auto y_at = [&](int which, int i) {
        return (uint16_t*)p.y[which] + b * p.y_sb[which] + (int64_t)s * p.y_ss[which] + col0 +
               head_ofs(p, hb + i, p.y_sh[which], p.y_sg[which]);
    };

    if constexpr (kCopy) {
        // Pack mode: every load of the block (q, k and the copied tensor) is
        // issued before any arithmetic; the shard is short, so this is where
        // the memory parallelism comes from.
        i32x4 raw[2][kChunk], rawc[kChunk];
        const uint16_t* xc = (const uint16_t*)p.xc + b * p.xc_sb + (int64_t)s * p.xc_ss + col0;
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
#pragma unroll
            for (int which = 0; which < 2; ++which) {
                raw[which][i] = i32x4{0, 0, 0, 0};
                if (i < nh && on) raw[which][i] = __builtin_nontemporal_load(x_at(which, i));
            }
            if (i < nh && on) rawc[i] = __builtin_nontemporal_load((const i32x4*)(xc + (int64_t)(hb + i) * p.xc_sh));
        }
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            float wv[8], wp[8];
            if (on) load_w8(p.w[which], col0, wf, wv);
            if (on && rot) load_w8(p.w[which], src * 8, wf, wp);
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                if (i >= nh) break;  // uniform
                row(raw[which][i], wv, wp, p.eps[which], y_at(which, i));
            }
        }
        uint16_t* yc = (uint16_t*)p.yc + b * p.yc_sb + (int64_t)s * p.yc_ss + col0;
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            if (i >= nh) break;  // uniform
            if (on) __builtin_nontemporal_store(rawc[i], (i32x4*)(yc + head_ofs(p, hb + i, p.yc_sh, p.yc_sg)));
        }
    } else {
        // Tensor by tensor, each tensor's loads issued first.
        for (int which = 0; which < p.n_tensors; ++which) {
            const bool second = which != 0;
            const void* w = second ? p.w[1] : p.w[0];
            const float eps = second ? p.eps[1] : p.eps[0];
            const int64_t xsh = second ? p.x_sh[1] : p.x_sh[0], ysh = second ? p.y_sh[1] : p.y_sh[0];
            const int64_t ysg = second ? p.y_sg[1] : p.y_sg[0];
            const uint16_t* xt = (const uint16_t*)(second ? p.x[1] : p.x[0]) + b * (second ? p.x_sb[1] : p.x_sb[0]) +
                                 (int64_t)s * (second ? p.x_ss[1] : p.x_ss[0]) + col0;
            uint16_t* yt = (uint16_t*)(second ? p.y[1] : p.y[0]) + b * (second ? p.y_sb[1] : p.y_sb[0]) +
                           (int64_t)s * (second ? p.y_ss[1] : p.y_ss[0]) + col0;
            float wv[8], wp[8];
            if (on) load_w8(w, col0, wf, wv);
            if (on && rot) load_w8(w, src * 8, wf, wp);
            i32x4 raw[kChunk];
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                raw[i] = i32x4{0, 0, 0, 0};
                if (i < nh && on) raw[i] = __builtin_nontemporal_load((const i32x4*)(xt + (int64_t)(hb + i) * xsh));
            }
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                if (i >= nh) break;  // uniform
                row(raw[i], wv, wp, eps, yt + head_ofs(p, hb + i, ysh, ysg));
            }
        }
    }
}

// Generic path (any even R <= D, any table alignment): one row per lane
// group, element-wise partner and table reads. Output heads may be grouped
// (the pack layout), and a copied third tensor goes along with the first
// tensor's rows (each (batch, token, head) once).
template <int L>
__global__ __launch_bounds__(kThreads) void qknorm_rope_generic_kernel(QkNormRopeParams p) {
    const int tid = threadIdx.x;
    const int j = tid % L;
    const RowRef ref = locate(p, blockIdx.x * (uint32_t)(kThreads / L) + (uint32_t)(tid / L));
    const int D = p.head_dim, R = p.rotary_dim, half = R >> 1;
    const int col0 = j * 8;
    const bool active = ref.ok && col0 < D;
    const void* w = ref.which ? p.w[1] : p.w[0];
    const bool wf = p.w_f32 != 0;
    float xv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (active) unpack8(*(const i32x4*)(ref.x + col0), xv);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
    if constexpr (L <= 16) {
        ss = group_sum<L>(ss);
    } else {
#pragma unroll
        for (int off = L / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, L);
    }
    if (!active) return;
    const float r = rsqrtf(ss / (float)D + (ref.which ? p.eps[1] : p.eps[0]));
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int col = col0 + e;
        float o = 0.f;
        if (col < D) {
            const float n = xv[e] * r * load_w(w, col, wf);
            if (col < R) {
                const bool first = col < half;
                const int pc = first ? col + half : col - half;
                const float pn = bf16_to_f32(ref.x[pc]) * r * load_w(w, pc, wf);
                const float rt = first ? -pn : pn;
                const float cv = p.cos[(int64_t)ref.s * p.table_stride + col];
                const float sv = p.sin[(int64_t)ref.s * p.table_stride + col];
                o = n * cv + rt * sv;
            } else {
                o = n;
            }
        }
        out[e] = o;
    }
    i32x4 packed;
#pragma unroll
    for (int e = 0; e < 4; ++e) packed[e] = (int)pack_bf16x2(out[2 * e], out[2 * e + 1]);
    *(i32x4*)(ref.y + col0) = packed;
    if (p.xc != nullptr && ref.which == 0) {
        const uint16_t* xc = (const uint16_t*)p.xc + (int64_t)ref.b * p.xc_sb + (int64_t)ref.s * p.xc_ss +
                             (int64_t)ref.h * p.xc_sh + col0;
        uint16_t* yc = (uint16_t*)p.yc + (int64_t)ref.b * p.yc_sb + (int64_t)ref.s * p.yc_ss +
                       head_ofs(p, (int)ref.h, p.yc_sh, p.yc_sg) + col0;
        *(i32x4*)yc = *(const i32x4*)xc;
    }
}

template <int L>
hipError_t launch_l(const QkNormRopeParams& p, bool fast, hipStream_t stream) {
    if (fast) {
        const int64_t batch = p.rows / ((int64_t)p.seqlen * p.n_tensors * p.heads);
        const int chunk = p.xc != nullptr ? kHeadChunkCopy : kHeadChunk;
        const dim3 grid((unsigned)((p.seqlen + kThreads / L - 1) / (kThreads / L)), (unsigned)((p.heads + chunk - 1) / chunk),
                        (unsigned)batch);
        if (p.xc != nullptr)
            hipLaunchKernelGGL((qknorm_rope_kernel<L, true>), grid, dim3(kThreads), 0, stream, p);
        else
            hipLaunchKernelGGL((qknorm_rope_kernel<L, false>), grid, dim3(kThreads), 0, stream, p);
    } else {
        const int64_t per_block = kThreads / L;
        const unsigned blocks = (unsigned)((p.rows + per_block - 1) / per_block);
        hipLaunchKernelGGL((qknorm_rope_generic_kernel<L>), dim3(blocks), dim3(kThreads), 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace

bool qknorm_rope_fast_path(const QkNormRopeParams& p) {
    if (p.rotary_dim == 0) return true;
    const bool aligned = ((uintptr_t)p.cos % 16 == 0) && ((uintptr_t)p.sin % 16 == 0) && (p.table_stride % 4 == 0);
    return (p.rotary_dim % 16 == 0) && aligned;
}

hipError_t launch_qknorm_rope(const QkNormRopeParams& p, hipStream_t stream) {
    if (p.rows <= 0) return hipSuccess;
    const bool fast = qknorm_rope_fast_path(p);
    int lanes = 1;
    while (lanes * 8 < p.head_dim) lanes <<= 1;
    switch (lanes) {
        case 1: return launch_l<1>(p, fast, stream);
        case 2: return launch_l<2>(p, fast, stream);
        case 4: return launch_l<4>(p, fast, stream);
        case 8: return launch_l<8>(p, fast, stream);
        case 16: return launch_l<16>(p, fast, stream);
        case 32: return launch_l<32>(p, fast, stream);
        case 64: return launch_l<64>(p, fast, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace h3a
