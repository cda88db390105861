// Projection GEMM for the H3 attention block (gfx950): Y = X W^T (+ bias),
// X (M tokens x K) and W (N features x K) bf16, both K-contiguous rows (the
// nn.Linear layout), fp32 accumulation on v_mfma_f32_32x32x16_bf16.
//
// The kernel computes the transposed product C^T = W X^T, so that after the
// MFMAs every lane holds one token and 64 of the 128 features of a head (the
// other 64 sit in lane ^ 32): a per-head epilogue (RMSNorm over the head,
// rotate-half RoPE pairing c with c +- 64) is then in-lane arithmetic plus
// one lane swap.
//
// Tiling: one workgroup = 8 waves = 256 features x 256 tokens; wave (wn, wm)
// owns features wn*128 .. +128 (one head) and tokens wm*64 .. +64. K advances
// 32 at a time through four LDS stages filled by HBM -> LDS DMA
// (buffer_load ... lds); the DMA of tile t+3 is issued after the barrier
// that frees its stage. LDS rows are 64 bytes; the 16-byte chunk c of row r
// sits at c ^ ((r >> 2) & 3), which keeps the fragment reads (32 rows x one
// chunk) free of bank conflicts.
#include <math.h>

#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kTN = 256;  // features per workgroup
constexpr int kTM = 256;  // tokens per workgroup
constexpr int kTK = 32;   // K per stage
constexpr int kStages = 4;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRowB = kTK * 2;          // LDS bytes per tile row
constexpr int kTileB = 256 * kRowB;     // 16 KB per operand per stage
constexpr int kLdsB = 2 * kStages * kTileB;

typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

__global__ __launch_bounds__(kThreads, 2) void proj_gemm_kernel(ProjGemmParams p) {
    __shared__ __attribute__((aligned(1024))) char smem[kLdsB];
    char* const wst = smem;                      // W stages
    char* const xst = smem + kStages * kTileB;   // X stages
    const lds_char* const lds = (const lds_char*)smem;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave >> 2, wm = wave & 3;
    const int l32 = lane & 31, hi = lane >> 5;

    // Workgroups go round-robin over the 8 XCDs; renumber them so each XCD
    // runs consecutive tiles, and order tiles in groups of kGroupM token
    // tiles x all feature tiles (token tile fastest): the ~32 workgroups an
    // XCD runs at once then cover 8 token tiles x 4 feature tiles and share
    // each X tile 4 ways and each W tile 8 ways in that XCD's L2.
    constexpr int kGroupM = 8;
    const int nb = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, per = nb >> 3, rem = nb & 7;
    const int tile = xcd * per + min(xcd, rem) + local;
    const int n_tiles = (p.n + kTN - 1) / kTN;
    const int in_group = kGroupM * n_tiles;
    const int first_m = (tile / in_group) * kGroupM;
    const int group_m = min(p.m_tiles - first_m, kGroupM);
    const int mt = first_m + (tile % in_group) % group_m, nt = (tile % in_group) / group_m;
    const int n0 = nt * kTN, m0 = mt * kTM;

    const char* wb = (const char*)p.w + (int64_t)n0 * p.w_rs;
    const char* xb = (const char*)p.x + (int64_t)m0 * p.x_rs;
    const int n_rows = min(kTN, p.n - n0), m_rows = min(kTM, p.m - m0);
    const i32x4 rw = make_rsrc_words(wb, (uint32_t)((n_rows - 1) * (int64_t)p.w_rs + p.k * 2));
    const i32x4 rx = make_rsrc_words(xb, (uint32_t)((m_rows - 1) * (int64_t)p.x_rs + p.k * 2));

    // DMA map: wave w fills rows 32w .. 32w+31 of each operand tile with two
    // 16-row loads; lane L writes LDS chunk (L & 3) of row r0 + (L >> 2),
    // which holds the tile's chunk (L & 3) ^ swz(row).
    uint32_t dw[2], dx[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = (wave * 2 + i) * 16 + (lane >> 2);
        const int chunk = ((lane & 3) ^ swz(r)) << 4;
        dw[i] = (uint32_t)(r * p.w_rs + chunk);
        dx[i] = (uint32_t)(r * p.x_rs + chunk);
    }
    const int nk = p.k / kTK;
    auto dma = [&](int kt) {
        kt = min(kt, nk - 1);  // past the end: reload the last tile into an unread stage
        const int stage = kt & (kStages - 1);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lw = (uint32_t)(uintptr_t)(const lds_char*)(wst + stage * kTileB + (wave * 2 + i) * 16 * kRowB);
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lw), "v"(dw[i] + kt * kRowB), "s"(rw)
                         : "memory");
            const uint32_t lx = (uint32_t)(uintptr_t)(const lds_char*)(xst + stage * kTileB + (wave * 2 + i) * 16 * kRowB);
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lx), "v"(dx[i] + kt * kRowB), "s"(rx)
                         : "memory");
        }
    };
    // Fragment of 32 rows starting at row0 of operand `op` (0: W, 1: X), K
    // substep ks (16 K): lane reads row row0 + l32, logical chunk 2*ks + hi.
    auto frag = [&](int op, int stage, int row0, int ks) {
        const int r = row0 + l32;
        const int off = (op * kStages + stage) * kTileB + r * kRowB + (((2 * ks + hi) ^ swz(r)) << 4);
        return *(const lds_bf16x8*)(lds + off);
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};

    // Pipeline: iteration kt issues the DMA of tile kt+3 (into the stage
    // tile kt-1 used), runs the 8 MFMAs of K substep 0 while reading the
    // fragments of substep 1, then the 8 MFMAs of substep 1. Before its
    // closing barrier it waits for its own DMA of tile kt+1, so after the
    // barrier tile kt+1 is complete and its substep-0 fragments are read
    // there, ahead of the next iteration's first MFMA.
    bf16x8 wf[2][4], xf[2][2];
    auto read_frags = [&](int stage, int ks) {
#pragma unroll
        for (int a = 0; a < 4; ++a) wf[ks][a] = frag(0, stage, wn * 128 + a * 32, ks);
#pragma unroll
        for (int b = 0; b < 2; ++b) xf[ks][b] = frag(1, stage, wm * 64 + b * 32, ks);
    };
    dma(0);
    dma(1);
    dma(2);
    wait_vmcnt<8>();  // tile 0 landed
    barrier();
    read_frags(0, 0);
    for (int kt = 0; kt < nk; ++kt) {
        const int stage = kt & (kStages - 1);
        dma(kt + 3);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int a = t >> 1, b = t & 1;
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[0][a], xf[0][b], acc[a][b], 0, 0, 0);
            if (t < 4) wf[1][t] = frag(0, stage, wn * 128 + t * 32, 1);
            else if (t < 6) xf[1][t - 4] = frag(1, stage, wm * 64 + (t - 4) * 32, 1);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int a = t >> 1, b = t & 1;
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[1][a], xf[1][b], acc[a][b], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        wait_vmcnt<8>();  // tile kt+1 landed (kt+2, kt+3 may be in flight)
        barrier();        // ... for every wave; stage kt is no longer read
        if (kt + 1 < nk) read_frags((kt + 1) & (kStages - 1), 0);
    }
    wait_vmcnt<0>();  // no DMA may land after the workgroup ends

    // Epilogue: lane holds token m0 + wm*64 + b*32 + l32 and, per feature
    // block a, features wn*128 + a*32 + 8*g + 4*hi + e (g < 4, e < 4) in
    // acc[a][b][4g + e].
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int m = m0 + wm * 64 + b * 32 + l32;
        if (m >= p.m) continue;
        char* yrow = (char*)p.y + (int64_t)m * p.y_rs;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn * 128 + a * 32 + 8 * g + 4 * hi;
                if (n >= p.n) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = acc[a][b][4 * g + e];
                    if (p.bias != nullptr) v[e] += p.bias_f32 ? ((const float*)p.bias)[n + e]
                                                              : bf16_to_f32(((const uint16_t*)p.bias)[n + e]);
                }
                i32x2 w;
                w.x = (int)pack_bf16x2(v[0], v[1]);
                w.y = (int)pack_bf16x2(v[2], v[3]);
                *(i32x2*)(yrow + n * 2) = w;
            }
    }
}

}  // namespace

hipError_t launch_proj_gemm(const ProjGemmParams& p, hipStream_t stream) {
    const int64_t tiles = (int64_t)p.m_tiles * ((p.n + kTN - 1) / kTN);
    if (tiles <= 0) return hipSuccess;
    hipLaunchKernelGGL(proj_gemm_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

int proj_gemm_tile_m() { return kTM; }
int proj_gemm_tile_k() { return kTK; }

}  // namespace h3a
