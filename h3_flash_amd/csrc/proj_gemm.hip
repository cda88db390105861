// Projection GEMM of the H3 attention block with the q/k RMSNorm + RoPE
// prologue as its epilogue (gfx950).
//
//   y[m, f] = sum_k x[m, k] * w[f, k] (+ bias[f])            (nn.Linear)
//   q / k sections: per (token m, head of 128 features) the result, rounded
//   to bf16 as the module's linear outputs it, is RMS-normalised in fp32,
//   scaled by the norm weight and rotated (rotate-half RoPE over the first R
//   features, table row m mod seqlen), then rounded to bf16 again: the
//   reference's order of a projection followed by fused_qknorm_rope; v and
//   out-projection sections are stored as they are.
//
// x (M tokens x K) and w (N features x K) are bf16 with K contiguous (the
// nn.Linear layout). The product is computed transposed, C^T = W X^T, on
// v_mfma_f32_16x16x32_bf16: the W fragment is the A operand (16 features x
// 32 K) and the X fragment the B operand (32 K x 16 tokens), so every lane of
// the result holds one token and 4 consecutive features per 16-feature block.
//
// Tiling: one workgroup = 4 waves = 256 features x 256 tokens, one wave per
// SIMD. Wave (wn, wm) owns features wn*128 .. +128 (one head) and tokens
// wm*128 .. +128: 8 x 8 MFMA blocks, 256 fp32 accumulators per lane (the
// accumulation registers), 16 fragment reads of 1 KB per 64 MFMAs.
//
// K advances 64 at a time through two LDS buffers of 32 KB per operand,
// filled HBM -> LDS by buffer_load ... lds (16 bytes per lane, no VGPR
// staging; each load covers whole 128-byte lines of 8 rows). LDS rows are 128
// bytes; the 16-byte chunk c of row r sits at c ^ ((r >> 1) & 7), so the 16
// rows a quarter-wave's fragment read touches hit 16 distinct bank groups.
// One barrier per K step of 64, in its middle: before it the wave waits for
// its own DMA of the next K step (issued during the previous step's second
// half, about 2,000 MFMA cycles earlier) and for its reads of the current
// buffer; after it the next step's fragments are read, and the step after
// next is loaded into the buffer just released, under the second half's
// MFMAs.
#include <math.h>

#include "common.h"
#include "kernels.h"

namespace h3a {
namespace {

constexpr int kPT = 256;                  // tile extent in features and in tokens
constexpr int kPK = 64;                   // K per stage (two MFMA K steps of 32)
constexpr int kPStages = 2;
constexpr int kPWaves = 4;
constexpr int kPThreads = kPWaves * 64;
constexpr int kPRow = kPK * 2;            // LDS bytes per tile row
constexpr int kPTile = kPT * kPRow;       // 32 KB per operand per stage
constexpr int kPXBase = kPStages * kPTile;  // X stages follow the W stages
constexpr int kPLds = 2 * kPStages * kPTile;
constexpr int kPDmaPerOp = kPT * kPRow / 1024 / kPWaves;  // 1 KB loads per wave per operand and stage
static_assert(kPDmaPerOp == 8, "DMA map below assumes eight loads per operand");

typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) float lds_f32;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// vmcnt(N) and lgkmcnt(0): the wave's own DMA loads beyond the newest N have
// landed and its LDS reads have completed.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// acc += A B on v_mfma_f32_16x16x32_bf16 with the accumulator pinned to the
// accumulation registers: with the builtin, the 256 accumulators of a lane
// are split between VGPRs and AGPRs and copied around the loop back edge.
__device__ __forceinline__ void mfma_acc(f32x4& acc, const bf16x8& a, const bf16x8& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// acc = A B (the first K step of a tile: no accumulator to read).
__device__ __forceinline__ void mfma_first(f32x4& acc, const bf16x8& a, const bf16x8& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
}

// Section i of the launch, selected field by field (indexing the kernel
// argument with a runtime index would copy the whole argument block into
// private memory).
__device__ __forceinline__ ProjSection section(const ProjGemmParams& p, int i) {
    ProjSection s = p.sec[0];
    if (i == 1) s = p.sec[1];
    if (i == 2) s = p.sec[2];
    return s;
}

// Tile t of the grouped order: groups of kGroupM token tiles x every feature
// tile, token tile fastest.
struct TileCoord {
    int sec;   // section of the feature tile
    int f0;    // first feature of the tile, within the section
    int m0;    // first token of the tile
};
constexpr int kGroupM = 2;
__device__ __forceinline__ TileCoord tile_coord(const ProjGemmParams& p, int tile) {
    const int in_group = kGroupM * p.n_tiles;
    const int first_m = (tile / in_group) * kGroupM;
    const int group_m = min(p.m_tiles - first_m, kGroupM);
    const int mt = first_m + (tile % in_group) % group_m;
    int nt = (tile % in_group) / group_m;
    int sec = 0;
    if (p.n_sections > 1 && nt >= p.sec[0].tiles) {
        nt -= p.sec[0].tiles;
        sec = 1;
        if (p.n_sections > 2 && nt >= p.sec[1].tiles) {
            nt -= p.sec[1].tiles;
            sec = 2;
        }
    }
    return TileCoord{sec, nt * kPT, mt * kPT};
}

// Where one tile's operands come from: the W and X buffer resources (based at
// the tile's first row; rows past the section or the token range are outside
// their records and load as zeros) and the per-lane part of the W offsets.
struct TileSrc {
    i32x4 rw, rx;
    uint32_t dw[2];
    int32_t w_rs;
};

// Epilogue LDS use: the output rows of RoPE sections, over the stage memory
// once the K loop is done: per wave 128 tokens x 256 bytes, the 8-byte chunk
// c of row r at c ^ (r mod 32), so that the 16 rows of a quarter-wave's
// writes fall in distinct bank pairs.
constexpr int kPOutWave = 128 * 256;
// RoPE epilogue with partners in other lanes: per wave, one token block's
// bf16 projection rows (16 tokens x 256 bytes), past the stage memory.
constexpr int kPRowsWave = 16 * 256;
constexpr int kPSmem = kPLds + kPWaves * kPRowsWave;
static_assert(kPWaves * kPOutWave <= kPLds, "output rows fit the stage memory");
static_assert(kPSmem <= 160 * 1024, "LDS of one workgroup");

// Epilogue of one tile: bias, then per section mode the plain value or the
// RMSNorm + norm weight + RoPE of each 128-feature head, rounded once to
// bf16. RoPE sections, and every section of a launch with RoPE sections or
// 16 KiB output rows (p.stage_plain), put their values into the wave's LDS
// rows first, which then go out as non-temporal 16-byte stores (4 token rows
// of 256 bytes per instruction); the others store straight from registers
// (lane pairs trade halves so each lane holds 8 consecutive features). The waves work
// independently (no barrier); `active` is false for the wave whose head
// lies past the section. The RoPE tables are in the rotate-half form
// (columns c and c + R/2 equal), so only their first R/2 columns are read,
// each lane loading its own token's values into registers one token block
// ahead.
__device__ __forceinline__ void epilogue(const ProjGemmParams& p, const TileCoord& tc, const f32x4 (&acc)[8][8],
                                         int wave, int wn, int wm, int lane, char* smem) {
    // Opaque here, so that no lane-derived value of the epilogue is hoisted
    // and held (or spilled) across the K loop.
    asm volatile("" : "+v"(lane));
    const ProjSection sec = section(p, tc.sec);
    // Lane l holds, for token block b (token wm*128 + 16b + (l & 15)) and
    // feature block a, features wn*128 + 16a + 4*(l >> 4) + e in acc[a][b][e]:
    // 32 of a head's 128 features; lanes l ^ 16, l ^ 32 and l ^ 48 hold the
    // other 96.
    const int f_head = tc.f0 + wn * 128;  // first feature of this wave's head, within the section
    const bool active = f_head < sec.n;   // false: the half of a 128-feature last tile past the section
    const bool norm = sec.mode != 0;
    const int R = norm ? p.rotary_dim : 0;
    const int fl = 4 * (lane >> 4);
    const int j16 = lane & 15;
    const int f_safe = active ? f_head : 0;
    const int seqlen = p.seqlen;
    const int m_head = tc.m0 + wm * 128;  // first token of the wave

    // RoPE tables straight into registers: for token block b the lane loads,
    // from its token's rows (wrapped per sequence), the first-half columns
    // 16*ta + fl .. +3 of cos and sin for each rotated block pair ta. The
    // loads of block b+1 are issued before block b is computed; the RoPE
    // path issues no stores until its rows are complete, so each wait is for
    // the tables alone (one counter covers loads and stores).
    const uint32_t tab_bytes = (uint32_t)((int64_t)seqlen * p.table_stride * 4);
    const auto rcos = make_rsrc(p.cos, tab_bytes);
    const auto rsin = make_rsrc(p.sin, tab_bytes);
    const uint32_t row_bytes = (uint32_t)(p.table_stride * 4);
    auto tab_offset = [&](int b) __attribute__((always_inline)) {
        int s = m_head + 16 * b + j16;
        s = s < seqlen ? s : s % seqlen;
        return (uint32_t)s * row_bytes + (uint32_t)fl * 4u;
    };
    const bool rope = R > 0;
    const bool staged = rope || p.stage_plain != 0;  // rows go out through LDS

    // Bias and norm weight of the lane's features (bf16, widened to fp32).
    const bool has_bias = sec.bias != nullptr;
    float bias[8][4], nw[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        const i32x2 br = has_bias ? *(const i32x2*)((const uint16_t*)sec.bias + f_safe + 16 * a + fl) : i32x2{0, 0};
        const i32x2 wr = norm ? *(const i32x2*)((const uint16_t*)sec.norm_w + 16 * a + fl) : i32x2{0, 0};
        bias[a][0] = __uint_as_float((uint32_t)br.x << 16);
        bias[a][1] = __uint_as_float((uint32_t)br.x & 0xffff0000u);
        bias[a][2] = __uint_as_float((uint32_t)br.y << 16);
        bias[a][3] = __uint_as_float((uint32_t)br.y & 0xffff0000u);
        nw[a][0] = __uint_as_float((uint32_t)wr.x << 16);
        nw[a][1] = __uint_as_float((uint32_t)wr.x & 0xffff0000u);
        nw[a][2] = __uint_as_float((uint32_t)wr.y << 16);
        nw[a][3] = __uint_as_float((uint32_t)wr.y & 0xffff0000u);
    }

    // bias, then RMSNorm over the head (sum of squares in-lane, then over
    // lanes l ^ 16 and l ^ 32) and the norm weight. Norm sections first round
    // the projection to bf16, as the module's linear outputs it, so the norm
    // and RoPE see the values the reference's separate steps see
    // (dense_fa4.py:123-140, transformer.py:146-173); rounding only once, at
    // the end, moves the LSE of the attention that follows by up to about
    // 2e-3 against that order.
    auto normed = [&](int b, float (&v)[8][4], auto norm_c) __attribute__((always_inline)) {
#pragma unroll
        for (int a = 0; a < 8; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[a][e] = acc[a][b][e] + bias[a][e];
        if constexpr (decltype(norm_c)::value) {
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const uint32_t r = pack_bf16x2(v[a][e], v[a][e + 1]);
                    v[a][e] = __uint_as_float(r << 16);
                    v[a][e + 1] = __uint_as_float(r & 0xffff0000u);
                }
            // Four partial sums (over e), added at the end: short dependency
            // chains for a lone wave.
            float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int e = 0; e < 4; ++e) s4[e] += v[a][e] * v[a][e];
            float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
            auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
            ss = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
            const f32x2 h = halves(ss);
            ss = h[0] + h[1];
            const float r = rsqrtf(ss * (1.0f / 128.0f) + sec.eps);
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[a][e] = (v[a][e] * r) * nw[a][e];
        }
    };
    lds_char* const orow = (lds_char*)smem + wave * kPOutWave;
    // Direct stores (sections without RoPE) go through a resource over this
    // wave's 128 token rows of its head: rows past the launch's tokens lie
    // outside its records and are dropped, and a wave whose head is past the
    // section gets no records at all, so no store needs a branch. f_pair:
    // byte offset of the lane's 8 features within a 32-feature group.
    // (Base and size go through readfirstlane: uniform, but the compiler
    // would otherwise keep the resource in VGPRs and wrap every store in a
    // waterfall loop.)
    const int rows_valid = active ? max(0, min(128, p.m - m_head)) : 0;
    const uint64_t ybase = (uint64_t)(uintptr_t)((const char*)sec.y + (int64_t)m_head * sec.y_rs + (int64_t)f_safe * 2);
    const uint32_t ybytes = rows_valid > 0 ? (uint32_t)((rows_valid - 1) * sec.y_rs + 256) : 0u;
    const auto yout = make_rsrc(
        (const void*)(uintptr_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(ybase >> 32)) << 32) |
                                 (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ybase)),
        (uint32_t)__builtin_amdgcn_readfirstlane((int)ybytes));
    const uint32_t f_pair = (uint32_t)((((lane >> 4) & 1) ? 16 : 0) + 4 * ((lane >> 4) & 2)) * 2u;
    // R a multiple of 32: every RoPE partner (c +- R/2, R/2 a multiple of 16)
    // is held by the same lane, feature block a pairing with a +- R/32, and
    // both use the table columns of block a mod R/32.
    auto in_lane = [&](auto rh_c, auto norm_c) __attribute__((always_inline)) {
        constexpr int rh = decltype(rh_c)::value, ra = 2 * rh;  // half of the rotated blocks, all of them
        constexpr int nt = rh > 0 ? rh : 1;
        f32x4 tcv[2][nt], tsv[2][nt];
        auto load_regs = [&](int b) __attribute__((always_inline)) {
            const uint32_t o = tab_offset(b);
#pragma unroll
            for (int ta = 0; ta < rh; ++ta) {
                tcv[b & 1][ta] = __builtin_bit_cast(f32x4, buf_load16(rcos, o + 64u * ta));
                tsv[b & 1][ta] = __builtin_bit_cast(f32x4, buf_load16(rsin, o + 64u * ta));
            }
        };
        if constexpr (ra > 0) load_regs(0);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            if constexpr (ra > 0) {
                if (b + 1 < 8) load_regs(b + 1);
            }
            float v[8][4];
            normed(b, v, norm_c);
            const int r = 16 * b + j16;
            if (ra == 0 && !staged) {
                // No tables to wait for: stores go out directly. Lanes l and
                // l ^ 16 (feature groups q, q ^ 1) trade one of two feature
                // blocks 2j, 2j+1 (permlane16_swap exchanges the first
                // operand of the odd lane with the second of the even one),
                // so that the even lane holds 8 consecutive features of
                // block 2j and the odd lane of block 2j+1: one 16-byte store
                // each, 64 contiguous bytes per token.
                const uint32_t row_off = (uint32_t)r * (uint32_t)sec.y_rs;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t p0x = pack_bf16x2(v[2 * j][0], v[2 * j][1]), p0y = pack_bf16x2(v[2 * j][2], v[2 * j][3]);
                    const uint32_t p1x = pack_bf16x2(v[2 * j + 1][0], v[2 * j + 1][1]);
                    const uint32_t p1y = pack_bf16x2(v[2 * j + 1][2], v[2 * j + 1][3]);
                    const auto sx = __builtin_amdgcn_permlane16_swap(p0x, p1x, false, false);
                    const auto sy = __builtin_amdgcn_permlane16_swap(p0y, p1y, false, false);
                    const i32x4 w{(int)sx[0], (int)sy[0], (int)sx[1], (int)sy[1]};
                    __builtin_amdgcn_raw_buffer_store_b128(w, yout, (int)(row_off + (uint32_t)(64 * j) + f_pair), 0, 0);
                }
                continue;
            }
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                float y[4];
                if (a < ra) {
                    const int pa = a < rh ? a + rh : a - rh;
                    const int ta = a < rh ? a : a - rh;
                    const f32x4 cw = tcv[b & 1][ta], sw = tsv[b & 1][ta];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float rot = a < rh ? -v[pa][e] : v[pa][e];
                        y[e] = v[a][e] * cw[e] + rot * sw[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) y[e] = v[a][e];
                }
                const i32x2 w{(int)pack_bf16x2(y[0], y[1]), (int)pack_bf16x2(y[2], y[3])};
                *(__attribute__((address_space(3))) i32x2*)(orow + r * 256 + ((((4 * a + (lane >> 4)) ^ r) & 31) << 3)) = w;
            }
        }
    };
    // Any other even R, or tables read at every rotated column: the partner
    // c +- R/2 of feature c is in general held by another lane of the token,
    // at another position. The norm starts from the bf16-rounded projection,
    // so the token's projection row is exact in bf16: it goes into the
    // wave's LDS row of the token (feature f at byte 2f, past the stage
    // memory), each lane reads its partners' values back, normalises them
    // with the token's r (the same in the 4 lanes of a token) and the
    // partner's norm weight, and reads cos / sin at its own columns. A
    // wave's LDS operations run in order: every lane's row writes precede
    // the reads, and a block's reads precede the next block's writes (the
    // memory clobbers keep the compiler from moving one past the other).
    lds_char* const prows = (lds_char*)smem + kPLds + wave * kPRowsWave;
    auto cross_lane = [&]() __attribute__((always_inline)) {
        const int rh = R >> 1;
        float wpart[8][4];  // norm weight at the partner column
#pragma unroll
        for (int a = 0; a < 8; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = 16 * a + fl + e;
                const int pc = c < rh ? c + rh : c - rh;
                wpart[a][e] = c < R ? bf16_to_f32(((const uint16_t*)sec.norm_w)[pc]) : 0.f;
            }
        // (Unrolled: the accumulators are registers, indexed by constants.)
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            float v[8][4];
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const uint32_t h2 = pack_bf16x2(acc[a][b][e] + bias[a][e], acc[a][b][e + 1] + bias[a][e + 1]);
                    v[a][e] = __uint_as_float(h2 << 16);
                    v[a][e + 1] = __uint_as_float(h2 & 0xffff0000u);
                }
            const int r = 16 * b + j16;
            lds_char* const prow = prows + j16 * 256;
            asm volatile("" ::: "memory");
#pragma unroll
            for (int a = 0; a < 8; ++a)
                *(__attribute__((address_space(3))) i32x2*)(prow + (16 * a + fl) * 2) =
                    i32x2{(int)pack_bf16x2(v[a][0], v[a][1]), (int)pack_bf16x2(v[a][2], v[a][3])};
            asm volatile("" ::: "memory");
            float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int e = 0; e < 4; ++e) s4[e] += v[a][e] * v[a][e];
            float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
            auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
            ss = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
            const f32x2 hs = halves(ss);
            ss = hs[0] + hs[1];
            const float rn = rsqrtf(ss * (1.0f / 128.0f) + sec.eps);
            int tok = m_head + r;
            tok = tok < seqlen ? tok : tok % seqlen;
            const uint32_t trow = (uint32_t)tok * row_bytes;
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int c = 16 * a + fl + e;
                    const float n = (v[a][e] * rn) * nw[a][e];
                    y[e] = n;
                    if (c < R) {
                        const int pc = c < rh ? c + rh : c - rh;
                        const float pp = bf16_to_f32(*(const __attribute__((address_space(3))) uint16_t*)(prow + pc * 2));
                        const float pn = (pp * rn) * wpart[a][e];
                        const uint32_t to = trow + (uint32_t)c * 4u;
                        const float cv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rcos, (int)to, 0, 0));
                        const float sv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsin, (int)to, 0, 0));
                        y[e] = n * cv + (c < rh ? -pn : pn) * sv;
                    }
                }
                const i32x2 w{(int)pack_bf16x2(y[0], y[1]), (int)pack_bf16x2(y[2], y[3])};
                *(__attribute__((address_space(3))) i32x2*)(orow + r * 256 + ((((4 * a + (lane >> 4)) ^ r) & 31) << 3)) = w;
            }
        }
    };
    using Y = std::true_type;
    if (!norm) {
        in_lane(std::integral_constant<int, 0>{}, std::false_type{});
    } else if (R > 0 && p.rope_full_tables != 0) {
        cross_lane();
    } else {
        switch (R) {
            case 0: in_lane(std::integral_constant<int, 0>{}, Y{}); break;
            case 32: in_lane(std::integral_constant<int, 1>{}, Y{}); break;
            case 64: in_lane(std::integral_constant<int, 2>{}, Y{}); break;
            case 96: in_lane(std::integral_constant<int, 3>{}, Y{}); break;
            default: in_lane(std::integral_constant<int, 4>{}, Y{}); break;  // 128 (other widths: cross_lane)
        }
    }
    if (!active || !staged) return;  // the rows went out directly
    // Lane l moves bytes 16*(l & 15) .. +16 of token row 4*it + (l >> 4) (the
    // wave's LDS ops are ordered, so its own writes are visible here).
    char* const yb = (char*)sec.y + (int64_t)f_head * 2 + j16 * 16;
#pragma unroll 8
    for (int it = 0; it < 32; ++it) {
        const int r = 4 * it + (lane >> 4);
        const lds_char* const src = (const lds_char*)orow + r * 256;
        const i32x2 lo = *(const __attribute__((address_space(3))) i32x2*)(src + ((((2 * j16) ^ r) & 31) << 3));
        const i32x2 hi = *(const __attribute__((address_space(3))) i32x2*)(src + ((((2 * j16 + 1) ^ r) & 31) << 3));
        const int m = m_head + r;
        // Non-temporal: whole 256-byte row pieces that no later tile reads
        // (q and k of the 40-head block 3.5% faster; the direct stores'
        // 64-byte pieces measured slower this way and stay ordinary).
        if (m < p.m) __builtin_nontemporal_store(i32x4{lo.x, lo.y, hi.x, hi.y}, (i32x4*)(yb + (int64_t)m * sec.y_rs));
    }
}

__global__ __launch_bounds__(kPThreads, 1) void proj_gemm_kernel(ProjGemmParams p) {
    __shared__ __attribute__((aligned(1024))) char smem[kPSmem];
    const lds_char* const lds = (const lds_char*)smem;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave >> 1, wm = wave & 1;

    // One workgroup per tile. Workgroup b runs on XCD b mod 8 (round-robin
    // dispatch) as that XCD's (b / 8)-th; each XCD owns one contiguous range
    // of the grouped tile order, so the ~32 tiles an XCD runs at a time are
    // consecutive in it (about 2 token tiles x 16 feature tiles sharing their
    // X and W panels in the XCD's L2). (A persistent grid of one workgroup
    // per CU looping over its XCD's range measured from 1% faster to 4%
    // slower, and is not used.)
    const int total = p.m_tiles * p.n_tiles;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3;
    const int per = total >> 3, rem = total & 7;
    const int first = xcd * per + min(xcd, rem), end = first + per + (xcd < rem ? 1 : 0);
    const int tile = first + local;
    if (tile >= end) return;  // the grid is the tile count: never taken

    // DMA map: load i of a wave fills rows (8*wave + i)*8 .. +8 of an operand
    // tile; lane L writes LDS chunk (L & 7) of row r0 + (L >> 3), which holds
    // the row's 16-byte chunk (L & 7) ^ swz(row), swz(r) = (r >> 1) & 7 =
    // 4*(i & 1) + (L >> 4) for these rows. The per-lane part of the source
    // offset depends on the parity of i; the load's first row and the K step
    // go into the scalar offset.
    int chunk[2];
#pragma unroll
    for (int par = 0; par < 2; ++par) chunk[par] = ((lane & 7) ^ ((4 * par + (lane >> 4)) & 7)) << 4;
    uint32_t dx[2];
#pragma unroll
    for (int par = 0; par < 2; ++par) dx[par] = (uint32_t)((lane >> 3) * p.x_rs + chunk[par]);
    auto source = [&](const TileCoord& tc) __attribute__((always_inline)) {
        const ProjSection sec = section(p, tc.sec);
        const int n_rows = min(kPT, sec.n - tc.f0), m_rows = min(kPT, p.m - tc.m0);
        const char* const wb = (const char*)sec.w + (int64_t)tc.f0 * sec.w_rs;
        const char* const xb = (const char*)p.x + (int64_t)tc.m0 * p.x_rs;
        TileSrc s;
        s.rw = make_rsrc_words(wb, (uint32_t)((int64_t)(n_rows - 1) * sec.w_rs + p.k * 2));
        s.rx = make_rsrc_words(xb, (uint32_t)((int64_t)(m_rows - 1) * p.x_rs + p.k * 2));
        s.w_rs = (int32_t)sec.w_rs;
#pragma unroll
        for (int par = 0; par < 2; ++par) s.dw[par] = (uint32_t)((lane >> 3) * sec.w_rs + chunk[par]);
        return s;
    };
    const int nk = p.k / kPK;
    // Load j (0..15) of this wave's share of K step kt of a tile into
    // `stage`: j < 8 are W rows, j >= 8 X rows. buffer_load ... lds writes 16
    // bytes per lane to LDS address M0 + 16*lane; M0 needs one wait state
    // before the load reads it (the two scalar offset instructions give it).
    // The scalar offsets are formed in the asm itself, per load: hoisted out
    // of the loop they would hold 32 scalar registers.
    const uint32_t lds_wave = (uint32_t)(uintptr_t)(lds + wave * kPDmaPerOp * 8 * kPRow);
    auto dma1 = [&](i32x4 rw, i32x4 rx, uint32_t dw0, uint32_t dw1, int w_rs, int kt, int stage, int j)
                    __attribute__((always_inline)) {
        const int i = j & 7;
        const bool is_w = j < 8;
        const uint32_t row8 = (uint32_t)(8 * (is_w ? w_rs : (int)p.x_rs));  // bytes of 8 rows
        const uint32_t base = (uint32_t)(wave * kPDmaPerOp) * row8 + (uint32_t)(kt * kPRow);
        const uint32_t voff = is_w ? ((i & 1) ? dw1 : dw0) : dx[i & 1];
        uint32_t soff;
        if (is_w)
            asm volatile(
                "s_add_u32 m0, %1, %2\n\ts_mul_i32 %0, %3, %4\n\ts_add_u32 %0, %0, %5\n\t"
                "buffer_load_dwordx4 %6, %7, %0 offen lds"
                : "=&s"(soff)
                : "s"(lds_wave), "i"(stage * kPTile + i * 8 * kPRow), "s"(row8), "i"(i), "s"(base), "v"(voff), "s"(rw)
                : "memory");
        else
            asm volatile(
                "s_add_u32 m0, %1, %2\n\ts_mul_i32 %0, %3, %4\n\ts_add_u32 %0, %0, %5\n\t"
                "buffer_load_dwordx4 %6, %7, %0 offen lds"
                : "=&s"(soff)
                : "s"(lds_wave), "i"(kPXBase + stage * kPTile + i * 8 * kPRow), "s"(row8), "i"(i), "s"(base),
                  "v"(voff), "s"(rx)
                : "memory");
    };
    auto dma_src = [&](const TileSrc& s, int kt, int stage, int j) __attribute__((always_inline)) {
        dma1(s.rw, s.rx, s.dw[0], s.dw[1], s.w_rs, kt, stage, j);
    };

    // Fragment reads: lane l takes row (16*block + (l & 15)) of the wave's
    // operand rows and, for MFMA K step h of the stage, logical chunk
    // 4h + (l >> 4) (K 32h + 8*(l>>4) .. +8); swz(row) = ((l & 15) >> 1) & 7.
    const int sl = (lane >> 1) & 7;
    const int fo0 = (lane & 15) * kPRow + (((lane >> 4) ^ sl) << 4);
    const int fo1 = (lane & 15) * kPRow + (((4 + (lane >> 4)) ^ sl) << 4);
    const lds_char* const wfr0 = lds + wn * 128 * kPRow + fo0;
    const lds_char* const wfr1 = lds + wn * 128 * kPRow + fo1;
    const lds_char* const xfr0 = lds + kPXBase + wm * 128 * kPRow + fo0;
    const lds_char* const xfr1 = lds + kPXBase + wm * 128 * kPRow + fo1;

    f32x4 acc[8][8];
    bf16x8 fw[2][8], fx[2][8];

    // Fragments of MFMA K step h of the stage in LDS buffer `st` into set h.
    auto read1 = [&](int st, int h, int j) __attribute__((always_inline)) {
        const lds_char* const xf = h ? xfr1 : xfr0;
        const lds_char* const wf = h ? wfr1 : wfr0;
        if (j < 8)
            fx[h][j] = *(const lds_bf16x8*)(xf + st * kPTile + j * 16 * kPRow);
        else
            fw[h][j - 8] = *(const lds_bf16x8*)(wf + st * kPTile + (j - 8) * 16 * kPRow);
    };
    // 64 MFMAs of fragment set h, feature block major, token blocks snaking,
    // with `extra(t)` issued after MFMA t; `first`: the tile's first K step.
    auto mfma64 = [&](int h, bool first, auto&& extra) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 64; ++t) {
            const int a = t >> 3, b = (a & 1) ? 7 - (t & 7) : (t & 7);
            if (first)
                mfma_first(acc[a][b], fw[h][a], fx[h][b]);
            else
                mfma_acc(acc[a][b], fw[h][a], fx[h][b]);
            extra(t);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    {
        const TileCoord tc = tile_coord(p, tile);
        const TileSrc cur = source(tc);
        // The tile's first two K steps.
#pragma unroll
        for (int j = 0; j < 16; ++j) dma_src(cur, 0, 0, j);
#pragma unroll
        for (int j = 0; j < 16; ++j) dma_src(cur, 1, 1, j);
        wait_vm_lgkm<16>();  // K step 0 (own loads) landed
        barrier();
#pragma unroll
        for (int j = 0; j < 16; ++j) read1(0, 0, j);

        // K step kt in LDS buffer st = kt mod 2, its first-half fragments in
        // set 0. First half: MFMAs of set 0 while set 1 is read from the same
        // stage. Then the wave's DMA of K step kt+1 (issued during the
        // previous step) is waited for, with its reads of stage st; after the
        // barrier every wave's part of K step kt+1 is in LDS and buffer st is
        // no longer read by anyone. Second half: MFMAs of set 1 while K step
        // kt+1's first-half fragments are read into set 0 and K step kt2 =
        // kt+2 is loaded into buffer st. The tile's last two steps load
        // nothing, and the last reads nothing.
        auto step = [&](auto st_c, auto dma_c, auto last_c, bool first, int kt2) __attribute__((always_inline)) {
            constexpr int st = decltype(st_c)::value;
            constexpr int nst = st ^ 1;
            constexpr bool dma = decltype(dma_c)::value, last = decltype(last_c)::value;
            mfma64(0, first, [&](int t) __attribute__((always_inline)) {
                if ((t & 1) == 1 && t < 32) read1(st, 1, t >> 1);
            });
            wait_vm_lgkm<0>();
            barrier();
            mfma64(1, false, [&](int t) __attribute__((always_inline)) {
                if (!last && (t & 3) == 1) read1(nst, 0, t >> 2);
                if (dma && (t & 3) == 0) dma_src(cur, kt2, st, t >> 2);
            });
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using T = std::true_type;
        using F = std::false_type;
        // K is a multiple of two steps (checked by the caller), so the buffer
        // of every step is a compile-time constant.
        if (nk == 2) {
            step(I0{}, F{}, F{}, true, 0);
            step(I1{}, F{}, T{}, false, 0);
        } else {
            step(I0{}, T{}, F{}, true, 2);
            step(I1{}, T{}, F{}, false, 3);
            for (int kt = 2; kt < nk - 2; kt += 2) {
                step(I0{}, T{}, F{}, false, kt + 2);
                step(I1{}, T{}, F{}, false, kt + 3);
            }
            step(I0{}, F{}, F{}, false, 0);
            step(I1{}, F{}, T{}, false, 0);
        }
        // No load is in flight and no wave reads the stages any more (the
        // last step's barrier followed every wave's last fragment read). The
        // MFMAs are inline asm, outside the compiler's hazard tracking: give
        // the last ones time to write their results before they are read.
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        epilogue(p, tc, acc, wave, wn, wm, lane, smem);
    }
}

}  // namespace

hipError_t launch_proj_gemm(const ProjGemmParams& p, hipStream_t stream) {
    const int64_t tiles = (int64_t)p.m_tiles * p.n_tiles;
    if (tiles <= 0) return hipSuccess;
    hipLaunchKernelGGL(proj_gemm_kernel, dim3((unsigned)tiles), dim3(kPThreads), 0, stream, p);
    return hipGetLastError();
}

int proj_gemm_tile() { return kPT; }
int proj_gemm_k_multiple() { return kPK * kPStages; }

}  // namespace h3a
