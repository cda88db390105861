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
//   * K/V tiles of 64 keys are double-buffered through LDS: tile j+1 is read
//     from HBM (128-bit buffer loads) into VGPRs while tile j is consumed,
//     then written to the other LDS stage behind one barrier per tile;
//   * V is transposed while it is staged (V^T rows of 64 keys) so that the
//     PV product O^T = V^T P^T takes its A operand with 64-bit LDS reads and
//     its B operand (P^T, bf16) straight from the S^T accumulators;
//   * softmax runs in the exp2 domain with fp32 running max / sum; the running
//     max is only raised when a tile exceeds it by more than 2^8, so the O
//     rescale is skipped for almost every tile.
#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kD = 128;           // head dim
constexpr int kBM = 128;          // query rows per workgroup
constexpr int kBN = 64;           // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kKRow = kD * 2 + 16;    // LDS bytes per K row (pad: 4 banks)
constexpr int kVRow = kBN * 2 + 8;    // LDS bytes per V^T row
constexpr int kKBytes = kBN * kKRow;  // 17408
constexpr int kVBytes = kD * kVRow;   // 17408
constexpr int kStage = kKBytes + kVBytes;
constexpr int kLdsBytes = 2 * kStage;
constexpr float kRescaleThreshold = 8.0f;  // log2 units

static_assert(kThreads == 256, "staging maps assume 256 threads");

__device__ __forceinline__ uint32_t span_bytes(int rows, int row_bytes) {
    return rows > 0 ? (uint32_t)((rows - 1) * row_bytes + kD * 2) : 0u;
}

__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];

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

    // Staging maps. K: thread owns rows (tid>>4) + 16*i, 16-byte chunk tid&15.
    // V: thread owns keys 4*(tid>>4) .. +3, head dims 8*(tid&15) .. +7.
    const int st_row = tid >> 4;
    const int st_chk = tid & 15;
    i32x4 kreg[4], vreg[4];

    auto load_tile = [&](int n0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            kreg[i] = buf_load16(rk, (uint32_t)((n0 + st_row + 16 * i) * p.k_rs + st_chk * 16));
#pragma unroll
        for (int r = 0; r < 4; ++r)
            vreg[r] = buf_load16(rv, (uint32_t)((n0 + 4 * st_row + r) * p.v_rs + st_chk * 16));
    };
    auto store_tile = [&](int stage) {
        char* kl = smem + stage * kStage;
        char* vl = kl + kKBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *(i32x4*)(kl + (st_row + 16 * i) * kKRow + st_chk * 16) = kreg[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int dw = e >> 1;
            const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
            i32x2 pr;
            pr.x = (int)__builtin_amdgcn_perm((uint32_t)vreg[1][dw], (uint32_t)vreg[0][dw], sel);
            pr.y = (int)__builtin_amdgcn_perm((uint32_t)vreg[3][dw], (uint32_t)vreg[2][dw], sel);
            *(i32x2*)(vl + (st_chk * 8 + e) * kVRow + st_row * 8) = pr;
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
    float m_run = -INFINITY;  // running max of raw scores for this lane's query
    float l_run = 0.f;        // this lane's partial sum (its half of the keys)
    const float c = p.scale_log2;

    const int ntiles = (sk + kBN - 1) / kBN;
    if (ntiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();

    for (int j = 0; j < ntiles; ++j) {
        const int n0 = j * kBN;
        const bool more = j + 1 < ntiles;
        if (more) load_tile(n0 + kBN);

        const char* kl = smem + (j & 1) * kStage;
        const char* vl = kl + kKBytes;

        // S^T (64 keys x 32 queries) = K_tile Q^T
        f32x16 s[2];
#pragma unroll
        for (int nb2 = 0; nb2 < 2; ++nb2) {
            s[nb2] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                bf16x8 a = *(const bf16x8*)(kl + (nb2 * 32 + l32) * kKRow + ks * 32 + hi * 16);
                s[nb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[ks], s[nb2], 0, 0, 0);
            }
        }
        // Keys past the end of the sequence (ragged last tile) get -inf.
        if (n0 + kBN > sk) {
#pragma unroll
            for (int nb2 = 0; nb2 < 2; ++nb2)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = n0 + nb2 * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                    if (key >= sk) s[nb2][r] = -INFINITY;
                }
        }

        // Online softmax (exp2 domain).
        float mx = s[0][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[0][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[1][r]);
        {
            f32x2 pr = halves(mx);
            mx = fmaxf(pr.x, pr.y);
        }
        const float m_new = fmaxf(m_run, mx);
        const bool need = (m_new - m_run) * c > kRescaleThreshold;
        if (__builtin_amdgcn_ballot_w64(need)) {
            const float m_use = need ? m_new : m_run;
            const float alpha = fast_exp2((m_run - m_use) * c);
            m_run = m_use;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        }
        const float mc = m_run * c;
        float lsum = 0.f;
#pragma unroll
        for (int nb2 = 0; nb2 < 2; ++nb2)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = fast_exp2(__builtin_fmaf(s[nb2][r], c, -mc));
                s[nb2][r] = pv;
                lsum += pv;
            }
        l_run += lsum;

        // P^T fragments: k-step cc covers keys 16*cc .. +15 and is made of
        // accumulator registers 8*(cc&1) .. +7 of s[cc>>1].
        bf16x8 pf[4];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const int nb2 = cc >> 1, rb = (cc & 1) * 8;
            f32x8 t;
#pragma unroll
            for (int i = 0; i < 8; ++i) t[i] = s[nb2][rb + i];
            pf[cc] = __builtin_convertvector(t, bf16x8);
        }

        // O^T (128 dims x 32 queries) += V^T P^T
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const char* vrow = vl + (db * 32 + l32) * kVRow;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int key = cc * 16 + hi * 4;
                i32x2 lo = *(const i32x2*)(vrow + key * 2);
                i32x2 hi2 = *(const i32x2*)(vrow + (key + 8) * 2);
                i32x4 av = {lo.x, lo.y, hi2.x, hi2.y};
                oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), pf[cc],
                                                                  oacc[db], 0, 0, 0);
            }
        }

        if (more) store_tile((j + 1) & 1);
        __syncthreads();
    }

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
