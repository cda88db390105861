// Dense non-causal attention forward for gfx950 (MI355X), bf16 in / bf16 out,
// fp32 log-sum-exp. Semantics follow the FlashAttention-4 call made by the
// reference adapter (src/h3_flash/runtime/attention/dense_fa4.py:74-80,145):
// O = softmax(scale * Q K^T) V over the full key range of each (batch, head),
// or of each packed segment when cu_seqlens are given.
//
// Tiling (one workgroup = 4 waves = 128 query rows of one head):
//   * each wave keeps 32 query rows resident in VGPRs as the B operand of
//     S^T = K Q^T (v_mfma_f32_32x32x16_bf16). Computing S transposed puts one
//     query column per lane, so the row max / row sum of the online softmax
//     are in-lane reductions plus one v_permlane32_swap across wave halves;
//   * K and V tiles of 64 keys are staged key-major in LDS, double-buffered:
//     while tile j is consumed, tiles j+1 (V) / j+2 (K) are read from HBM with
//     128-bit buffer loads into VGPRs and written behind one barrier per tile;
//   * the PV product O^T = V^T P^T takes its A operand with the gfx950
//     transpose read ds_read_b64_tr_b16 (four keys of one head-dim column per
//     lane) and its B operand (P^T, bf16) straight from the S^T accumulators;
//   * software pipeline: iteration j issues the QK^T MFMAs of tile j+1, then
//     the PV MFMAs of tile j, and the softmax VALU work of tile j+1 (which only
//     depends on the first group) overlaps the second group;
//   * softmax runs in the exp2 domain with fp32 running max / sum; the running
//     max is only raised when a tile exceeds it by more than 2^8, so the O
//     rescale is skipped for almost every tile.
// LDS row strides are padded so that every access pattern is bank-conflict
// free: K rows (272 B) shift 4 banks per row for the 16-lane b128 reads; V rows
// (320 B) shift 16 banks per row for the 4-row x 32-byte transpose reads.
#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kD = 128;           // head dim
constexpr int kBM = 128;          // query rows per workgroup
constexpr int kBN = 64;           // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kKRow = kD * 2 + 16;    // LDS bytes per K row
constexpr int kVRow = kD * 2 + 64;    // LDS bytes per V row
constexpr int kKBytes = kBN * kKRow;  // 17408
constexpr int kVBytes = kBN * kVRow;  // 20480
constexpr int kLdsBytes = 2 * (kKBytes + kVBytes);
constexpr float kRescaleThreshold = 8.0f;  // log2 units

static_assert(kThreads == 256, "staging maps assume 256 threads");

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ uint32_t span_bytes(int rows, int row_bytes) {
    return rows > 0 ? (uint32_t)((rows - 1) * row_bytes + kD * 2) : 0u;
}

// Four bf16 of one head-dim column: within each 16-lane group lane i receives
// element (i & 3) of the 8-byte chunks addressed by lanes 4j + (i >> 2).
__device__ __forceinline__ i32x2 read_tr(const char* p) {
    s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    return __builtin_bit_cast(i32x2, v);
}

__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];
    char* const kst = smem;                // K stages 0, 1
    char* const vst = smem + 2 * kKBytes;  // V stages 0, 1

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hi = lane >> 5;   // wave half
    const int l32 = lane & 31;

    // Workgroups are dispatched round-robin over the 8 XCDs. Renumber them so
    // that the workgroups resident on one XCD at the same time are
    // consecutive query tiles of one head and share its K/V in that XCD's L2.
    const int nb = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, per = nb >> 3, rem = nb & 7;
    const int logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
    const int qt = logical % p.n_qtiles;
    const int rest = logical / p.n_qtiles;
    const int h = rest % p.heads;
    const int grp = rest / p.heads;

    int b = grp, q0 = 0, k0 = 0, sq = p.seqlen_q, sk = p.seqlen_k;
    if (p.cu_q != nullptr) {
        // Segment bounds are clamped to the packed rows, so no cu_seqlens
        // content can move an access outside the tensors.
        b = 0;
        q0 = min(max(p.cu_q[grp], 0), p.seqlen_q);
        sq = min(max(p.cu_q[grp + 1], q0), p.seqlen_q) - q0;
        k0 = min(max(p.cu_k[grp], 0), p.seqlen_k);
        sk = min(max(p.cu_k[grp + 1], k0), p.seqlen_k) - k0;
    }
    const int m0 = qt * kBM;
    if (m0 >= sq) return;  // whole workgroup: tile beyond this segment

    const char* qb = (const char*)p.q + 2 * (b * p.q_sb + h * p.q_sh) + (int64_t)q0 * p.q_rs;
    const char* kb = (const char*)p.k + 2 * (b * p.k_sb + h * p.k_sh) + (int64_t)k0 * p.k_rs;
    const char* vb = (const char*)p.v + 2 * (b * p.v_sb + h * p.v_sh) + (int64_t)k0 * p.v_rs;
    const auto rq = make_rsrc(qb, span_bytes(sq, p.q_rs));
    const auto rk = make_rsrc(kb, span_bytes(sk, p.k_rs));
    const auto rv = make_rsrc(vb, span_bytes(sk, p.v_rs));

    // Q fragment: lane holds query row (m0 + 32*wave + l32), head dims
    // 16*ks + 8*hi .. +8 for ks = 0..7 (B operand of S^T = K Q^T).
    const int mq = m0 + wave * 32 + l32;
    bf16x8 qf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        i32x4 raw = buf_load16(rq, (uint32_t)(mq * p.q_rs + ks * 32 + hi * 16));
        qf[ks] = __builtin_bit_cast(bf16x8, raw);
    }

    // Staging map (K and V alike): thread owns rows (tid>>4) + 16*i of a tile
    // and their 16-byte chunk tid&15; 16 lanes cover one 256-byte row.
    const int st_row = tid >> 4;
    const int st_chk = tid & 15;
    i32x4 kreg[4], vreg[4];
    auto load_k = [&](int tile) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            kreg[i] = buf_load16(rk, (uint32_t)((tile * kBN + st_row + 16 * i) * p.k_rs + st_chk * 16));
    };
    auto load_v = [&](int tile) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            vreg[i] = buf_load16(rv, (uint32_t)((tile * kBN + st_row + 16 * i) * p.v_rs + st_chk * 16));
    };
    auto store_k = [&](int stage) {
        char* dst = kst + stage * kKBytes + st_row * kKRow + st_chk * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) *(i32x4*)(dst + 16 * i * kKRow) = kreg[i];
    };
    auto store_v = [&](int stage) {
        char* dst = vst + stage * kVBytes + st_row * kVRow + st_chk * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) *(i32x4*)(dst + 16 * i * kVRow) = vreg[i];
    };

    const float c = p.scale_log2;
    const int ntiles = (sk + kBN - 1) / kBN;

    // S^T (64 keys x 32 queries) = K_tile Q^T from K stage `stage`.
    auto qk = [&](int stage, f32x16* s) {
        const char* kl = kst + stage * kKBytes + l32 * kKRow + hi * 16;
#pragma unroll
        for (int nb2 = 0; nb2 < 2; ++nb2) {
            s[nb2] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                bf16x8 a = *(const bf16x8*)(kl + nb2 * 32 * kKRow + ks * 32);
                s[nb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[ks], s[nb2], 0, 0, 0);
            }
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
    float m_run = -INFINITY;  // running max of raw scores for this lane's query
    float l_run = 0.f;        // this lane's partial sum (its half of the keys)
    bf16x8 pf[4];             // P^T of the tile waiting for its PV product

    // Online softmax of tile `tile` held in s: updates m_run / l_run and
    // writes the bf16 P^T fragments; returns the factor alpha by which the
    // accumulated O must be rescaled (exactly 1 unless the running max rose
    // by more than the threshold). Branch-free, so the scheduler can overlap
    // it with the PV MFMAs issued before it.
    auto softmax = [&](f32x16* s, int tile, bool ragged) -> float {
        if (ragged) {  // last tile: keys past the end get -inf
            const int n0 = tile * kBN;
#pragma unroll
            for (int nb2 = 0; nb2 < 2; ++nb2)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = n0 + nb2 * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                    if (key >= sk) s[nb2][r] = -INFINITY;
                }
        }
        float mx = fmaxf(s[0][0], s[1][0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[0][r], s[1][r]));
        {
            f32x2 pr = halves(mx);
            mx = fmaxf(pr.x, pr.y);
        }
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new - m_run) * c > kRescaleThreshold ? m_new : m_run;
        const float alpha = fast_exp2((m_run - m_use) * c);
        m_run = m_use;
        const float mc = m_use * c;
        float lsum = 0.f;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            // k-step cc covers keys 16*cc .. +15: accumulator registers
            // 8*(cc&1) .. +7 of s[cc>>1]
            f32x8 t;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pv = fast_exp2(__builtin_fmaf(s[cc >> 1][(cc & 1) * 8 + i], c, -mc));
                t[i] = pv;
                lsum += pv;
            }
            pf[cc] = __builtin_convertvector(t, bf16x8);
        }
        l_run = __builtin_fmaf(l_run, alpha, lsum);
        return alpha;
    };
    // Keep the exp/convert work in its block, next to the PV MFMAs it
    // overlaps, instead of letting it sink past the rescale branch. (An empty
    // volatile asm also closes the scheduling region.)
    auto pin_softmax = [&]() {
        asm volatile("" ::"v"(pf[0]), "v"(pf[1]), "v"(pf[2]), "v"(pf[3]), "v"(l_run));
    };
    auto rescale = [&](float alpha) {
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        }
    };

    // O^T (128 dims x 32 queries) += V^T P^T from V stage `stage`.
    auto pv = [&](int stage) {
        // transpose-read addresses: lane (l & 15) of a 16-lane group reads key
        // row (l & 15) >> 2 and dims 4*(l & 3) .. +3 of its group's 16 columns
        const int g = lane & 15;
        const char* vl = vst + stage * kVBytes + ((g >> 2) + hi * 4) * kVRow + (((lane >> 4) & 1) * 16 + 4 * (g & 3)) * 2;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const char* a0 = vl + (cc * 16) * kVRow + db * 64;
                i32x2 lo = read_tr(a0);
                i32x2 up = read_tr(a0 + 8 * kVRow);
                i32x4 av = {lo.x, lo.y, up.x, up.y};
                oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), pf[cc], oacc[db],
                                                                  0, 0, 0);
            }
    };

    // Pipeline: before iteration j, P_j is in registers, K_{j+1} and V_j are
    // in LDS. Iteration j computes S_{j+1} and O += V_j P_j, then the softmax
    // of S_{j+1}, while K_{j+2} and V_{j+1} travel HBM -> VGPR -> LDS.
    const bool ragged = ntiles * kBN > sk;
    if (ntiles > 0) {
        load_k(0);
        load_v(0);
        store_k(0);
        store_v(0);
        if (ntiles > 1) {
            load_k(1);
            store_k(1);
        }
        __syncthreads();
        f32x16 s[2];
        qk(0, s);
        softmax(s, 0, ntiles == 1 && ragged);
        __syncthreads();  // K stage 0 is refilled in the first iteration
    }
    int j = 0;
    for (; j + 2 < ntiles; ++j) {  // steady state: tiles j+1 and j+2 exist
        load_k(j + 2);
        load_v(j + 1);
        f32x16 s[2];
        qk((j + 1) & 1, s);
        pv(j & 1);
        const float alpha = softmax(s, j + 1, false);
        // Issue order for the block above: the HBM loads, then each QK^T MFMA
        // behind its K fragment read, then each PV MFMA behind its two
        // transpose reads followed by a slice of the softmax VALU work, so the
        // softmax issues while the PV MFMAs execute.
        __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);  // VMEM read
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // VALU
        }
        pin_softmax();
        rescale(alpha);
        store_k(j & 1);
        store_v((j + 1) & 1);
        __syncthreads();
    }
    if (j + 1 < ntiles) {  // j = ntiles - 2: the last tile is loaded, no K beyond
        load_v(j + 1);
        f32x16 s[2];
        qk((j + 1) & 1, s);
        pv(j & 1);
        const float alpha = softmax(s, j + 1, ragged);
        pin_softmax();
        rescale(alpha);
        store_v((j + 1) & 1);
        __syncthreads();
        ++j;
    }
    if (j < ntiles) pv(j & 1);  // j = ntiles - 1

    // Epilogue: combine the two halves' partial sums, normalise, store.
    {
        f32x2 pr = halves(l_run);
        l_run = pr.x + pr.y;
    }
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    if (mq < sq) {
        char* ob = (char*)p.o + 2 * (b * p.o_sb + h * p.o_sh) + (int64_t)(q0 + mq) * p.o_rs;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = db * 32 + i * 8 + hi * 4;
                i32x2 w;
                w.x = (int)pack_bf16x2(oacc[db][i * 4 + 0] * inv, oacc[db][i * 4 + 1] * inv);
                w.y = (int)pack_bf16x2(oacc[db][i * 4 + 2] * inv, oacc[db][i * 4 + 3] * inv);
                *(i32x2*)(ob + d * 2) = w;
            }
        if (p.lse != nullptr && hi == 0) {
            const float lse = l_run > 0.f ? (m_run * c + __log2f(l_run)) * 0.69314718055994531f : -INFINITY;
            p.lse[b * p.lse_sb + h * p.lse_sh + q0 + mq] = lse;
        }
    }
}

}  // namespace

int attn_fwd_block_m() { return kBM; }

hipError_t launch_attn_fwd(const AttnParams& p, hipStream_t stream) {
    const int64_t blocks = (int64_t)p.n_qtiles * p.heads * p.n_groups;
    if (blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace h3a
