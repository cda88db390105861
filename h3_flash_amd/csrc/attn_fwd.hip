// Dense non-causal attention forward for gfx950 (MI355X), bf16 in / bf16 out,
// fp32 log-sum-exp. Semantics follow the FlashAttention-4 call made by the
// reference adapter (src/h3_flash/runtime/attention/dense_fa4.py:74-80,145):
// O = softmax(scale * Q K^T) V over the full key range of each (batch, head),
// or of each packed segment when cu_seqlens are given.
//
// Tiling: one workgroup = 8 waves = 256 query rows of one head, one workgroup
// per CU (two waves per SIMD).
//   * each wave keeps 32 query rows resident in VGPRs as the B operand of
//     S^T = K Q^T (v_mfma_f32_32x32x16_bf16). Computing S transposed puts one
//     query column per lane, so the row max / row sum of the online softmax
//     are in-lane reductions plus one v_permlane32_swap across wave halves;
//   * K and V tiles of 64 keys go HBM -> LDS directly (buffer_load ... lds,
//     16 bytes per lane, no VGPR staging) into four LDS stages each; one
//     barrier per tile, after each wave's own loads of the previous
//     iteration are complete (s_waitcnt vmcnt), so every load has a whole
//     iteration to land;
//   * the PV product O^T = V^T P^T takes its A operand with the gfx950
//     transpose read ds_read_b64_tr_b16 (four keys of one head-dim column per
//     lane) and its B operand (P^T, bf16) straight from the S^T accumulators;
//   * three-tile software pipeline (hand scheduled, sched_barrier fenced):
//     iteration j issues the 16 QK^T MFMAs of tile j+2, then the 16 PV MFMAs
//     of tile j, with K / V fragments read four MFMAs ahead, and spreads the
//     softmax of tile j+1 (VALU and exp2) in slices between all 32 MFMAs;
//   * softmax runs in the exp2 domain, p = exp2(s*c - mc), with an fp32 row
//     sum. The offset mc is the first tile's max; later tiles reduce no max:
//     the row sum bounds every p, and when it passes 2^16 the offset rises
//     by the sum's binary exponent and P, O and l are scaled by that power
//     of two, exactly. A tile whose row sum passes 2^64 (a score more than
//     ~64 log2 units above the offset, up to p = inf) is recomputed from K
//     in global memory against its exact max.
// LDS rows are 256 bytes, unpadded; the 16-byte chunk c of row r is stored at
// chunk c ^ swz(r), swz(r) = 4*(r & 3) + ((r >> 2) & 3). Both read patterns are
// then bank-conflict free: the K reads (16 consecutive rows, one chunk) and the
// V transpose reads (4 consecutive rows x 4 chunks per 32 lanes).
#include <atomic>
#include <type_traits>

#include "common.h"
#include "kernels.h"

// Workspace of h3a_attn_fwd_noalloc: the partial results (bf16 O, fp32 LSE) of the tail's
// key-range pieces and the tail's counter, for callers that cannot allocate.
// Every GPU the library runs on holds its own copy until the process ends.
// Host code never passes `scratch` itself (on the host it names a shadow
// variable, not device memory): attn_static_scratch looks up this device's
// copy with hipGetSymbolAddress and kernels take that address.
static __device__ __align__(256) char scratch[h3a::kStaticScratchBytes];

namespace h3a {
namespace {

constexpr int kD = 128;            // head dim
constexpr int kBM = 256;           // query rows per workgroup
constexpr int kBN = 64;            // keys per tile
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kStages = 4;
constexpr int kRow = kD * 2;       // LDS bytes per K / V row
constexpr int kTile = kBN * kRow;  // 16384
constexpr int kLdsBytes = 2 * kStages * kTile;
constexpr int kDmaPerTile = kBN / (kWaves * 4);  // 4-row DMA loads per wave per tile
constexpr float kSumLimit = 65536.0f;            // row-sum bound of the fast softmax path
// Row sum past which a tile's softmax is recomputed against its exact max. A
// p of 2^127 * (2 - 2^-8) or more is finite in fp32 but rounds to inf in bf16,
// and a rescale by 2^-ex with ex > 126 is subnormal; below 2^64 neither occurs.
constexpr float kRecomputeLimit = 0x1p64f;
// Rows a K / V buffer resource of the wide forms spans from its base: the
// pipeline prologue loads tiles 0..4 from the view's first tile; the main
// loop rebases the K resource at the one tile each load reads and moves a
// token-major V window on every four tiles (loads up to tile j+6 from base
// j). So 32-bit buffer offsets only ever cover one window of the view,
// however long the view is. The host accepts a view when kWindowRows of its
// rows span less than 2^31 bytes.
constexpr int kWindowRows = kBN * 9;
constexpr int kPersistMaxQTiles = 16;  // longest segment of a persistent launch: 4,096 rows
constexpr int kQueuePieces = 4;                  // key-range pieces per tile of a dynamic tail
// Fewest key tiles in such a piece: each piece pays a pipeline fill and
// drain and a partial result, which short pieces do not recover (8 x 8,192-row
// segments at 5 heads cut into pieces of 32 key tiles ran 5% slower).
constexpr int kQueueMinKeyTiles = 48;
// Key tiles from which a 4-way queued split is graded (its small pieces keep
// 32 key tiles or more).
constexpr int kGradedMinKeyTiles = 256;

static_assert(kDmaPerTile == 2, "vmcnt accounting below assumes 2 K + 2 V loads per iteration");
static_assert(kStages == 4, "the pipeline below is unrolled over four stages");

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

__device__ __forceinline__ uint32_t span_bytes(int rows, int row_bytes) {
    return rows > 0 ? (uint32_t)((rows - 1) * row_bytes + kD * 2) : 0u;
}

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// LDS chunk swizzle of a d-major V tile (128-byte rows): 16 consecutive rows
// read at one logical chunk hit 16 different 16-byte bank groups.
__device__ __forceinline__ int vswz(int r) { return (r >> 1) & 7; }

// Key order of the S^T rows with a d-major V: bits 2 and 3 of the row index
// swapped. A lane then holds keys 8*hi .. 8*hi + 7 of every 16-key step of
// P^T, which one ds_read_b128 of a d-major V row matches.
__device__ __forceinline__ int keyperm(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// First key of packed segment s (its first key row k0, clamped) in the
// d-major V of a varlen launch: k0 rounded up to a multiple of 64, plus 64
// per earlier segment. Segments never overlap there when the offsets ascend,
// and every segment stays inside the rows of roundup(seqlen_k, 64) +
// 64 * num_segments keys whatever the offsets hold.
__device__ __forceinline__ int vt_segment_start(int k0, int s) { return (k0 + kBN - 1) / kBN * kBN + kBN * s; }

// Four bf16 of one head-dim column: within each 16-lane group lane i receives
// element (i & 3) of the 8-byte chunks addressed by lanes 4j + (i >> 2).
__device__ __forceinline__ i32x2 read_tr(const lds_char* p) {
    s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    return __builtin_bit_cast(i32x2, v);
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that leaves the memory counters to the caller: the LDS
// DMA loads in flight are waited for explicitly (wait_vmcnt) before it.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// The lane's index within its wave, counted by the hardware (v_mbcnt): a
// value that can be taken again after a long loop instead of being held in
// a register across it.
__device__ __forceinline__ int lane_from_hw() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// The launch arguments as the tail loop reads them: where they lie (the
// kernel-argument segment, through the scalar cache).
using KernArgs = const __attribute__((address_space(4))) AttnParams;

// The tile's LDS: one array however many copies of attn_tile a kernel holds.
__device__ __forceinline__ char* attn_lds() {
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
    return smem;
}

// One query tile (chunk < 0), or key-range piece `chunk` of `chunks` of a
// tile. A piece with a workspace slot (slot >= 0) writes normalised fp32
// partial O and LSE there for the merge; a whole tile, or a piece covering
// the tile's whole key range (slot < 0), writes O and LSE. All waves of the
// workgroup call it with the same arguments; it returns with no LDS DMA in
// flight.
// kWide: views whose span reaches 2^31 bytes. Their K / V buffer resources
// are rebased as the key loop moves on (a window of kWindowRows rows), so
// 32-bit offsets never cover more than one window. Shorter views keep one
// resource per view: the rebase needs scalar registers this kernel does not
// have to spare, so it is not paid where it is not needed.
// kVT: V is read from a d-major copy (p.vt: per (batch, head) 128 rows of
// keys, zero past the last key), so each PV fragment is one ds_read_b128
// instead of two transpose reads. The K rows of every 16-key group are then
// taken in the order that swaps bits 2 and 3 of the key index (keyperm), so
// that the eight keys a lane holds in P^T are consecutive.
// kPersist (packed launches without a work list, neither wide nor d-major
// V): qcarry holds Q across calls; `prefetched` says that the previous call
// already issued this tile's Q loads and its first K / V DMA, and next_tile
// (-1: none) is the tile whose first loads this call issues in its last two
// iterations. cu_cur and cu_next hold cu_q[s], cu_q[s + 1], cu_k[s],
// cu_k[s + 1] of this tile's and the next tile's segment, loaded by the
// caller one tile ahead. Returns whether it issued the next tile's loads.
template <bool kWide, bool kVT, bool kPersist = false, typename Params>
__device__ __forceinline__ bool attn_tile(Params& p, int tile, int chunk, int chunks, int slot,
                                          bool graded = false, bf16x8* qcarry = nullptr, bool prefetched = false,
                                          int next_tile = -1, const int* cu_cur = nullptr,
                                          const int* cu_next = nullptr, int wave_first = 0) {
    static_assert(!kPersist || (!kWide && !kVT), "persistent launches use the narrow token-major form");
    char* const smem = attn_lds();
    // V stages 0..3 first, then K stages 0..3: with a per-lane base in a VGPR
    // every fragment read offset then fits the 16-bit ds_read immediate.
    char* const vst = smem;
    char* const kst = smem + kStages * kTile;
    const lds_char* const lds = (const lds_char*)smem;

    // Opaque per call, so that no lane-derived value is hoisted out of the
    // piece loop in attn_fwd_kernel and held across it (that cost VGPRs and
    // spills).
    // The wide forms, short of registers, hold no copy of the work-item id
    // across calls: wave_first (the wave's first work item, a scalar the
    // kernel reads once) plus the lane.
    int tid = kWide ? wave_first + lane_from_hw() : (int)threadIdx.x;
    asm volatile("" : "+v"(tid));
    int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int hi = lane >> 5;  // wave half
    int l32 = lane & 31;
    // Key (within a 32-key block) of S^T row r.
    auto krowperm = [](int r) { return kVT ? keyperm(r) : r; };

    const int qt = tile % p.n_qtiles;
    const int rest = tile / p.n_qtiles;
    const int h = rest % p.heads;
    const int grp = rest / p.heads;

    int b = grp, q0 = 0, k0 = 0, sq = p.seqlen_q, sk = p.seqlen_k;
    int vpad = 0;  // key offset of this segment in the d-major V
    if (p.cu_q != nullptr) {
        // Segment bounds are clamped to the packed rows, so no cu_seqlens
        // content can move an access outside the tensors.
        b = 0;
        int cq0, cq1, ck0, ck1;
        if constexpr (kPersist) {
            cq0 = __builtin_amdgcn_readfirstlane(cu_cur[0]);
            cq1 = __builtin_amdgcn_readfirstlane(cu_cur[1]);
            ck0 = __builtin_amdgcn_readfirstlane(cu_cur[2]);
            ck1 = __builtin_amdgcn_readfirstlane(cu_cur[3]);
        } else {
            cq0 = p.cu_q[grp];
            cq1 = p.cu_q[grp + 1];
            ck0 = p.cu_k[grp];
            ck1 = p.cu_k[grp + 1];
        }
        q0 = min(max(cq0, 0), p.seqlen_q);
        sq = min(max(cq1, q0), p.seqlen_q) - q0;
        k0 = min(max(ck0, 0), p.seqlen_k);
        sk = min(max(ck1, k0), p.seqlen_k) - k0;
        if (kVT) vpad = vt_segment_start(k0, grp) - k0;
    }
    const int m0 = qt * kBM;
    if (m0 >= sq) return false;  // whole workgroup: tile beyond this segment
    if (chunk >= 0) {
        // Piece c of n covers key tiles [c*nkt/n, (c+1)*nkt/n). Graded
        // pieces (a queue's 4-way split of long key ranges) cover 3/8, 3/8,
        // 1/8 and 1/8 instead: the queue hands out every tile's first pieces
        // before any last one, so the pieces left at the end of the launch
        // are small and the CUs finish closer together.
        const int nkt = (sk + kBN - 1) / kBN;
        int kt0 = chunk * nkt / chunks, kt1 = (chunk + 1) * nkt / chunks;
        if (graded && chunks == 4 && nkt >= kGradedMinKeyTiles) {
            auto edge = [](int c) { return c < 2 ? 3 * c : c + 4; };  // 0, 3, 6, 7, 8 eighths
            kt0 = edge(chunk) * nkt / 8;
            kt1 = edge(chunk + 1) * nkt / 8;
        }
        k0 += kt0 * kBN;
        sk = min(sk - kt0 * kBN, (kt1 - kt0) * kBN);
    }

    // The Q resource starts at the tile's first query row; K / V resources
    // start at the first key row of their window (kWide) or of the view.
    const int q_first = kWide ? m0 : 0;  // first row of the Q resource, from the segment's
    const char* qb = (const char*)p.q + 2 * (b * p.q_sb + h * p.q_sh) + (int64_t)(q0 + q_first) * p.q_rs;
    const char* kb = (const char*)p.k + 2 * (b * p.k_sb + h * p.k_sh) + (int64_t)k0 * p.k_rs;
    // d-major V: key k0 of dim row 0 of this head; a head's block is 128 rows
    // of vt_rs bytes.
    const char* vb = kVT ? (const char*)p.vt + 2 * (b * p.vt_sb + h * p.vt_sh + (int64_t)(k0 + vpad))
                         : (const char*)p.v + 2 * (b * p.v_sb + h * p.v_sh) + (int64_t)k0 * p.v_rs;
    // The window of a K / V view starting at key tile j0 (kWide), or the
    // whole view: rows past the view's end are outside the range and load as
    // zeros.
    auto window = [&](const char* base, int row_bytes, int j0) {
        if constexpr (kWide)
            return make_rsrc_words(base + (int64_t)j0 * (kBN * row_bytes),
                                   span_bytes(min(sk - j0 * kBN, kWindowRows), row_bytes));
        else
            return make_rsrc_words(base, span_bytes(sk, row_bytes));
    };
    // The Q loads and the K / V DMA are written as inline asm, so the
    // compiler tracks none of them: it cannot tell the LDS stages apart and
    // would otherwise wait for every DMA in flight (vmcnt(0)) before the
    // first LDS read that follows one. Their completion is ordered explicitly
    // with wait_vmcnt, barriers and register pins below.
    const i32x4 rq = make_rsrc_words(qb, span_bytes(kWide ? min(sq - m0, kBM) : sq, p.q_rs));
    i32x4 rk = window(kb, p.k_rs, 0);
    // The d-major V resource ends at the end of this head's block: tiles past
    // the padded key range read the next dim row's keys (finite values that
    // meet P = 0) or, in the last row, zeros.
    i32x4 rv = kVT ? make_rsrc_words(vb, (uint32_t)(kD * p.vt_rs - 2 * (k0 + vpad))) : window(vb, p.v_rs, 0);
    // Moves a token-major V window (kWide) four key tiles on, to start at
    // tile j0: the 48-bit base of words 0-1 (stride bits zero) grows by
    // 4 * kBN rows; the range is recomputed from the rows left.
    auto advance = [&](i32x4& r, int row_bytes, int j0) {
        const uint64_t base = ((uint64_t)(uint32_t)r.y << 32 | (uint32_t)r.x) + (uint64_t)(4 * kBN) * (uint32_t)row_bytes;
        r.x = (int)(uint32_t)base;
        r.y = (int)((uint32_t)(base >> 32) & 0xffffu);
        r.z = (int)span_bytes(min(sk - j0 * kBN, kWindowRows), row_bytes);
    };

    // Q fragment: lane holds query row (m0 + 32*wave + l32), head dims
    // 16*ks + 8*hi .. +8 for ks = 0..7 (B operand of S^T = K Q^T).
    const int mq = m0 + wave * 32 + l32;
    bf16x8 qf_own[8];
    bf16x8(&qf)[8] = *(kPersist ? (bf16x8(*)[8])qcarry : &qf_own);
    const bool issue = !kPersist || !prefetched;  // false: the previous tile issued Q and the first K / V
    if (kPersist && issue) {
        // Q is carried across the loop of a persistent launch, where the
        // compiler may copy its registers: compiler-tracked loads, which it
        // waits for before any copy or use.
        const __amdgpu_buffer_rsrc_t rqb = make_rsrc(qb, span_bytes(sq, p.q_rs));
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rqb, (uint32_t)(mq * p.q_rs + ks * 32 + hi * 16)));
    } else if (issue) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            i32x4 raw;
            asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen"
                         : "=v"(raw)
                         : "v"((uint32_t)((mq - q_first) * p.q_rs + ks * 32 + hi * 16)), "s"(rq)
                         : "memory");
            qf[ks] = __builtin_bit_cast(bf16x8, raw);
        }
    }

    // DMA map: wave w fills rows 8w .. 8w+7 of a tile with two 4-row loads;
    // lane L writes LDS chunk (L & 15) of row r0 + (L >> 4), which holds the
    // tile's chunk (L & 15) ^ swz(row) of that key row. The per-lane byte
    // offset inside a tile is fixed; the tile's first row adds a uniform term.
    // Rows past the end of the view are out of the buffer's range: zeros.
    uint32_t dk[kDmaPerTile], dv[kDmaPerTile];
#pragma unroll
    for (int i = 0; i < kDmaPerTile; ++i) {
        const int r = (wave * kDmaPerTile + i) * 4 + (lane >> 4);
        const int chunk = ((lane & 15) ^ swz(r)) << 4;
        dk[i] = (uint32_t)(r * p.k_rs + chunk);
        dv[i] = (uint32_t)(r * p.v_rs + chunk);
        if constexpr (kVT) {
            // d-major V tile: 128 rows (head dims) of 128 bytes (64 keys); lane
            // L writes LDS chunk (L & 7) of row rt + (L >> 3), which holds the
            // row's 16-byte chunk (L & 7) ^ vswz(row).
            const int rt = (wave * kDmaPerTile + i) * 8 + (lane >> 3);
            dv[i] = (uint32_t)(rt * p.vt_rs + (((lane & 7) ^ vswz(rt)) << 4));
        }
    }
    // buffer_load ... lds writes 16 bytes per lane to LDS address M0 + 16*lane;
    // M0 needs one wait state before the load reads it. Nothing else in this
    // kernel uses M0 (it is a reserved register, so it is not listed as
    // clobbered). `tile` counts from the resource's first tile. An opaque
    // skip (a scalar the compiler cannot fold) is added to the lane offset at
    // the load itself, where a constant one would have the compiler hold
    // every (tile, load) sum in its own VGPR.
    auto dma1 = [&](const i32x4& rsrc, int row_bytes, const uint32_t* lanes, char* stage, int tile, int i,
                    bool opaque = false) {
        // A tile is kBN rows of row_bytes, or (d-major V, row_bytes 0) 2 * kBN
        // bytes along every dim row.
        uint32_t skip = (uint32_t)(tile * (row_bytes != 0 ? kBN * row_bytes : 2 * kBN));
        if (opaque) asm volatile("" : "+s"(skip));
        const uint32_t dst = (uint32_t)(uintptr_t)(const lds_char*)(stage + (wave * kDmaPerTile + i) * 4 * kRow);
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :
                     : "s"(dst), "v"(lanes[i] + skip), "s"(rsrc)
                     : "memory");
    };
    // Load i (of kDmaPerTile) of this wave's share of a K / V tile.
    auto dma_k1 = [&](int tile, int stage, int i) { dma1(rk, p.k_rs, dk, kst + stage * kTile, tile, i); };
    // (The token-major V of the wide forms is addressed per window of four
    // tiles, with opaque skips.)
    auto dma_v1 = [&](int tile, int stage, int i) {
        dma1(rv, kVT ? 0 : p.v_rs, dv, vst + stage * kTile, tile, i, kWide && !kVT);
    };
    auto dma_k = [&](int tile, int stage) {
#pragma unroll
        for (int i = 0; i < kDmaPerTile; ++i) dma_k1(tile, stage, i);
    };
    auto dma_v = [&](int tile, int stage) {
#pragma unroll
        for (int i = 0; i < kDmaPerTile; ++i) dma_v1(tile, stage, i);
    };

    // K fragment of QK^T MFMA t (key block t & 1, head-dim step t >> 1): row
    // 32*(t & 1) + l32, logical chunk 2*(t >> 1) + hi.
    // The swizzle only moves bits 4-7 of an in-row byte offset, so every
    // fragment address is a per-lane base XOR a per-step constant. K: offset
    // kbase ^ (32*ks) (+32 rows for the second key block).
    const int krow = kVT ? keyperm(l32) : l32;
    const int kbase = krow * kRow + ((hi ^ swz(krow)) << 4);
    // Transpose-read addresses of PV MFMA t (head-dim block db = t >> 2, key
    // step cc = t & 3): lane (g = l & 15) of a 16-lane group reads row
    // 16*cc + 4*hi + (g >> 2) (+8 for the upper four keys) and head dims
    // 32*db + 16*((l >> 4) & 1) + 4*(g & 3) .. +3. With swz(row) =
    // 4*(g >> 2) ^ hi ^ 2*upper, the offset is
    // 4096*cc + 2048*upper + (vbase ^ 64*db ^ 32*upper).
    int vbase;
    {
        const int g = lane & 15, jr = g >> 2, dgrp = (lane >> 4) & 1, u = (g & 3) >> 1;
        vbase = (4 * hi + jr) * kRow + ((32 * dgrp) ^ (16 * u) ^ (64 * jr) ^ (16 * hi)) + (g & 1) * 8;
    }

    const float c = p.scale_log2;
    const int ntiles = (sk + kBN - 1) / kBN;

    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
    // Exponent offset of this lane's query, log2 units: p = exp2(s*c - mc).
    // Set from the first tile's max, raised in whole steps when a tile's
    // row sum grows past kSumLimit.
    float mc = 0.f;
    float l_run = 0.f;        // this lane's partial sum (its half of the keys)

    // Per-lane LDS byte offsets of the K fragments (one per head-dim step)
    // and of the V transpose reads (one per head-dim block and key half); the
    // empty asm keeps each in a register so stage and step offsets become
    // instruction immediates.
    // d-major V (kVT): the A fragment of PV MFMA (db, cc) is row 32*db + l32,
    // logical chunk 2*cc + hi, stored at chunk (2*cc + hi) ^ vswz(l32): a
    // per-lane base XOR 32*cc, plus 4096*db.
    constexpr int kVofs = kVT ? 4 : 8;
    uint32_t kofs[8], vofs[kVofs];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        kofs[ks] = (uint32_t)(kStages * kTile + (kbase ^ (32 * ks)));
        asm volatile("" : "+v"(kofs[ks]));
    }
#pragma unroll
    for (int i = 0; i < kVofs; ++i) {
        if constexpr (kVT)
            vofs[i] = (uint32_t)((l32 * 2 * kBN + ((hi ^ vswz(l32)) << 4)) ^ (32 * i));
        else
            vofs[i] = (uint32_t)(vbase ^ (64 * (i >> 1)) ^ (32 * (i & 1)));
        asm volatile("" : "+v"(vofs[i]));
    }
    auto kread = [&](int stage, int t) {
        return *(const lds_bf16x8*)(lds + kofs[t >> 1] + (stage * kTile + (t & 1) * 32 * kRow));
    };
    // A fragment of PV MFMA (head-dim block db, 16-key step cc).
    auto vread = [&](int stage, int db, int cc) {
        if constexpr (kVT) {
            return *(const lds_bf16x8*)(lds + vofs[cc] + (stage * kTile + db * 32 * 2 * kBN));
        } else {
            const lds_char* a = lds + (stage * kTile + cc * 16 * kRow);
            const i32x2 lo = read_tr(a + vofs[2 * db]);
            const i32x2 up = read_tr(a + 8 * kRow + vofs[2 * db + 1]);
            return __builtin_bit_cast(bf16x8, i32x4{lo.x, lo.y, up.x, up.y});
        }
    };
    auto mask_tail = [&](f32x16& s0, f32x16& s1, int tile) {
        const int n0 = tile * kBN;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = n0 + krowperm((r >> 2) * 8 + hi * 4 + (r & 3));
            if (key >= sk) s0[r] = -INFINITY;
            if (key + 32 >= sk) s1[r] = -INFINITY;
        }
    };

    // Persistent launches: set once this tile has issued the next tile's
    // loads, Q into qf included (its last two iterations).
    bool pref = false;
    // Redo the softmax of a tile whose row sum passed kRecomputeLimit: S again from
    // K in global memory (its LDS stage may already hold a newer tile) and
    // the resident Q, then the exact max of the tile, a new offset at or
    // above it, and O and l rescaled to that offset. Leaves every p <= 1.
    const auto rk_plain = make_rsrc(kb, span_bytes(sk, p.k_rs));
    auto overflow = [&](int tile, bf16x8* pout, float& lsum) __attribute__((always_inline)) {
        // K rows of the tile, from a resource at the tile's first row (kWide)
        // or at the view's.
        const int first = kWide ? tile * kBN : 0;
        const auto rk_tile =
            kWide ? make_rsrc(kb + (int64_t)first * p.k_rs, span_bytes(min(sk - first, kBN), p.k_rs)) : rk_plain;
        f32x16 s2[2] = {f32x16{}, f32x16{}};
        bool q_resident = true;
        if constexpr (kPersist) q_resident = !pref;
        if (q_resident) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const uint32_t row = (uint32_t)(tile * kBN - first + 32 * (t & 1) + krow);
                const i32x4 raw = buf_load16(rk_tile, row * (uint32_t)p.k_rs + (t >> 1) * 32 + hi * 16);
                s2[t & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, raw), qf[t >> 1],
                                                                    s2[t & 1], 0, 0, 0);
            }
        } else if constexpr (kPersist) {
            // The last softmax of a persistent tile runs after qf took the
            // next tile's Q: this tile's Q fragments come from memory again.
            const __amdgpu_buffer_rsrc_t rq_cur = make_rsrc(qb, span_bytes(sq, p.q_rs));
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const bf16x8 qk = __builtin_bit_cast(bf16x8, buf_load16(rq_cur, (uint32_t)(mq * p.q_rs + ks * 32 + hi * 16)));
#pragma unroll
                for (int t = 2 * ks; t < 2 * ks + 2; ++t) {
                    const uint32_t row = (uint32_t)(tile * kBN - first + 32 * (t & 1) + krow);
                    const i32x4 raw = buf_load16(rk_tile, row * (uint32_t)p.k_rs + ks * 32 + hi * 16);
                    s2[t & 1] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, raw), qk, s2[t & 1], 0, 0, 0);
                }
            }
        }
        if ((tile + 1) * kBN > sk) mask_tail(s2[0], s2[1], tile);
        float mx = s2[0][0];
#pragma unroll
        for (int e = 1; e < 32; ++e) mx = fmaxf(mx, s2[e >> 4][e & 15]);
        const f32x2 pr = halves(mx);
        const float mc_new = fmaxf(mc, fmaxf(pr.x, pr.y) * c);
        const float alpha = fast_exp2(mc - mc_new);
        mc = mc_new;
        lsum = 0.f;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            i32x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = 8 * cc + 2 * i;
                const float a0 = fast_exp2(__builtin_fmaf(s2[e >> 4][e & 15], c, -mc));
                const float a1 = fast_exp2(__builtin_fmaf(s2[e >> 4][(e & 15) + 1], c, -mc));
                lsum += a0 + a1;
                w[i] = (int)pack_bf16x2(a0, a1);
            }
            pout[cc] = __builtin_bit_cast(bf16x8, w);
        }
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        l_run *= alpha;
    };

    // One pipeline iteration, three stages wide: the 16 QK^T MFMAs of a tile
    // (K stage kl) into s_out, the 16 PV MFMAs of an older tile (V stage vl,
    // P fragments pin), and the online softmax of the tile in between (s_in,
    // tile sm_tile) cut into one slice per MFMA, so its VALU work issues under
    // all 32 MFMAs: each slice exponentiates one or two scores and packs
    // them to bf16 into pout. Each part is
    // switched on by a std::true_type / std::false_type argument (the
    // pipeline prologue runs subsets). Keys past the end of the sequence
    // (ragged last tile, padding tiles) are masked to -inf.
    // kf carries the first four K fragments of an iteration's QK^T group; they
    // are read before the barrier that ends the previous iteration (kl_next
    // names their stage; -1: none) so the next MFMA group starts at once.
    bf16x8 kf[4];
    auto iterate = [&](auto qk_on, auto sm_on, auto pv_on, int kl, int vl, int sm_tile, f32x16* s_in, f32x16* s_out,
                       const bf16x8* pin, bf16x8* pout, int kl_next, auto&& hook) __attribute__((always_inline)) {
        constexpr bool kQK = decltype(qk_on)::value;
        constexpr int kSM = decltype(sm_on)::value;  // 0: none, 1: running offset, 2: first tile
        constexpr bool kPV = decltype(pv_on)::value;
        constexpr int kSlices = (kQK ? 16 : 0) + (kPV ? 16 : 0);
        static_assert(kSM == 0 || kSlices >= 16, "the softmax is spread over at least 16 slices");
        if constexpr (kSM) {
            if ((sm_tile + 1) * kBN > sk) {
                // A real branch, not per-element selects: only the last tiles take it.
                asm volatile("" ::: "memory");
                mask_tail(s_in[0], s_in[1], sm_tile);
            }
        }
        float lsum = 0.f, mx = 0.f;
        float pe[32];
        uint32_t pn[16];
        // Each slice exponentiates one score (two without the PV half)
        // against the offset mc, adds it to the fp32 row sum and packs pairs
        // to bf16. Only the first tile reduces its max (slices 0-1) to set mc.
        constexpr int kFirstExp = kSM == 2 ? 2 : 0;
        auto slice = [&](int k) __attribute__((always_inline)) {
            if constexpr (kSM == 2) {
                if (k == 0) {
                    mx = s_in[0][0];
#pragma unroll
                    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s_in[0][r]);
                } else if (k == 1) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_in[1][r]);
                    const f32x2 pr = halves(mx);
                    mc = fmaxf(pr.x, pr.y) * c;  // finite: tile 0 has a key
                }
            }
            if constexpr (kSM != 0) {
                if (k >= kFirstExp) {
                    const int e0 = ((k - kFirstExp) * 32) / (kSlices - kFirstExp);
                    const int e1 = ((k - kFirstExp + 1) * 32) / (kSlices - kFirstExp);
#pragma unroll
                    for (int e = e0; e < e1; ++e) {
                        // The sum and the bf16 pair take the previous score, so
                        // no instruction waits on the exp just issued (the
                        // order of the fp32 sum is unchanged).
                        pe[e] = fast_exp2(__builtin_fmaf(s_in[e >> 4][e & 15], c, -mc));
                        if (e >= 1) lsum = e == 1 ? pe[0] : lsum + pe[e - 1];  // fp32: l feeds the LSE
                        if (e >= 2 && !(e & 1)) pn[(e - 1) >> 1] = pack_bf16x2(pe[e - 2], pe[e - 1]);
                    }
                }
            }
        };
        bf16x8 vf[4];
        if constexpr (kQK) {
            s_out[0] = f32x16{};
            s_out[1] = f32x16{};
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                s_out[t & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t & 3], qf[t >> 1], s_out[t & 1], 0, 0, 0);
                if (t + 4 < 16) kf[t & 3] = kread(kl, t + 4);
                if (kPV && t >= 12) vf[t - 12] = vread(vl, t - 12, 0);
                hook(t);
                slice(t);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (kPV) {
            if constexpr (!kQK) {
#pragma unroll
                for (int t = 0; t < 4; ++t) vf[t] = vread(vl, t, 0);
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                oacc[t & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[t & 3], pin[t >> 2], oacc[t & 3], 0, 0, 0);
                if (t + 4 < 16) vf[t & 3] = vread(vl, (t + 4) & 3, (t + 4) >> 2);
                if (t >= 12 && kl_next >= 0) kf[t - 12] = kread(kl_next, t - 12);
                hook((kQK ? 16 : 0) + t);
                slice((kQK ? 16 : 0) + t);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (kSM != 0) {
            lsum += pe[31];
            pn[15] = pack_bf16x2(pe[30], pe[31]);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                pout[cc] = __builtin_bit_cast(bf16x8, i32x4{(int)pn[4 * cc], (int)pn[4 * cc + 1], (int)pn[4 * cc + 2],
                                                            (int)pn[4 * cc + 3]});
            // Keep the softmax work in its block, next to the MFMAs it
            // overlaps, instead of letting it sink into the branch below.
            asm volatile("" ::"v"(pout[0]), "v"(pout[1]), "v"(pout[2]), "v"(pout[3]), "v"(lsum));
            // Every p of the lane is at most its row sum. A sum past
            // kSumLimit (scores well above the offset) raises the offset of
            // the query by the sum's binary exponent, for both lanes of the
            // query: P, O and l are scaled by that power of two, exactly. O
            // holds this iteration's PV products, all at the old offset, and
            // the next PV adds this tile's P.
            if (__builtin_amdgcn_ballot_w64(lsum > kSumLimit)) {
                asm volatile("" ::: "memory");  // a real branch
                if (__builtin_amdgcn_ballot_w64(lsum > kRecomputeLimit)) {
                    asm volatile("" ::: "memory");
                    overflow(sm_tile, pout, lsum);
                }
                int ex = lsum > kSumLimit ? __builtin_amdgcn_frexp_expf(lsum) : 0;
                {
                    const f32x2 pr = halves(__int_as_float(ex));
                    ex = max(__float_as_int(pr.x), __float_as_int(pr.y));
                }
                const float alpha = __builtin_ldexpf(1.0f, -ex);
                mc += (float)ex;
                lsum *= alpha;
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    i32x4 w = __builtin_bit_cast(i32x4, pout[cc]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t u = (uint32_t)w[i];
                        w[i] = (int)pack_bf16x2(__uint_as_float(u << 16) * alpha,
                                                __uint_as_float(u & 0xffff0000u) * alpha);
                    }
                    pout[cc] = __builtin_bit_cast(bf16x8, w);
                }
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
                l_run *= alpha;
            }
            l_run += lsum;
        }
    };

    // Pipeline: K_t and V_t live in LDS stage t % 4. Iteration j issues the
    // QK^T of tile j+2, the softmax of tile j+1 and the PV of tile j, and the
    // DMA of K_{j+5} (into K_{j+1}'s stage) and V_{j+3} (into V_{j-1}'s); its
    // last PV steps already read the first K fragments of tile j+3. At its
    // end vmcnt(4) leaves only its own loads in flight, so after the barrier
    // every wave sees K_{j+4} and V_{j+2} (issued at iteration j-1), the
    // tiles iteration j+1 reads ahead. The loop runs a multiple of 4 iterations,
    // unrolled so that every stage offset is a compile-time constant and S
    // and P ping-pong between two register sets each; tiles past the end read
    // as zeros and are fully masked.
    f32x16 sa[2], sb[2];
    bf16x8 pfa[4], pfb[4];
    auto no_hook = [](int) {};
    constexpr std::integral_constant<int, 0> kNoSoftmax{};
    constexpr std::integral_constant<int, 1> kSoftmax{};
    constexpr std::integral_constant<int, 2> kFirstSoftmax{};
    const int nsteps = (ntiles + 3) & ~3;
    if (ntiles > 0) {
        if (issue) {
            dma_k(0, 0);
            dma_k(1, 1);
            dma_v(0, 0);
            dma_k(2, 2);
            dma_v(1, 1);
            dma_k(3, 3);
            dma_v(2, 2);
        }
        // Prefetched by the previous tile, in this order, before that
        // tile's O stores: the stores are younger, so each wait below only
        // gets stronger.
        wait_vmcnt<6 * kDmaPerTile>();  // Q and K_0 have landed
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) asm volatile("" : "+v"(qf[ks]));  // no Q use before the wait
        barrier();
#pragma unroll
        for (int t = 0; t < 4; ++t) kf[t] = kread(0, t);
        iterate(std::true_type{}, kNoSoftmax, std::false_type{}, 0, 0, 0, sb, sa, pfb, pfb, -1, no_hook);
        barrier();  // K stage 0 is free
        dma_k(4, 0);
        wait_vmcnt<6 * kDmaPerTile>();  // K_1 has landed
        barrier();
#pragma unroll
        for (int t = 0; t < 4; ++t) kf[t] = kread(1, t);
        iterate(std::true_type{}, kFirstSoftmax, std::false_type{}, 1, 0, 0, sa, sb, pfb, pfa, -1, no_hook);
        wait_vmcnt<2 * kDmaPerTile>();  // V_0, K_2, V_1 and K_3 too
        barrier();                      // and K stage 1 is free
#pragma unroll
        for (int t = 0; t < 4; ++t) kf[t] = kread(2, t);
    }
    // Persistent launches: the first PV-only iteration issues the next
    // tile's Q loads (Q's registers are dead after the last QK^T) and its
    // K_0..K_3 and V_0, V_1 DMA (the K stages and V stages 0, 1 are no longer
    // read), in the order of the prologue above; the second issues V_2 into
    // stage 2, which the first one's PV read. The vmcnt(0) first lets the
    // past-end DMA of this tile land before the same rows are written again.
    // The Q loads are compiler builtins, so the compiler waits for them
    // before any use or copy of their registers.
    i32x4 nrv{};
    auto prefetch = [&]() __attribute__((always_inline)) {
        if constexpr (kPersist) {
            if (next_tile < 0) return;
            const int nqt = next_tile % p.n_qtiles;
            const int nh = (next_tile / p.n_qtiles) % p.heads;
            const int nq0 = min(max(__builtin_amdgcn_readfirstlane(cu_next[0]), 0), p.seqlen_q);
            const int nsq = min(max(__builtin_amdgcn_readfirstlane(cu_next[1]), nq0), p.seqlen_q) - nq0;
            const int nk0 = min(max(__builtin_amdgcn_readfirstlane(cu_next[2]), 0), p.seqlen_k);
            const int nsk = min(max(__builtin_amdgcn_readfirstlane(cu_next[3]), nk0), p.seqlen_k) - nk0;
            const int nm0 = nqt * kBM;
            if (nm0 >= nsq || nsk <= 0) return;  // the next call issues nothing either
            wait_vmcnt<0>();
            const char* nqb = (const char*)p.q + 2 * (nh * p.q_sh) + (int64_t)nq0 * p.q_rs;
            const char* nkb = (const char*)p.k + 2 * (nh * p.k_sh) + (int64_t)nk0 * p.k_rs;
            const char* nvb = (const char*)p.v + 2 * (nh * p.v_sh) + (int64_t)nk0 * p.v_rs;
            const __amdgpu_buffer_rsrc_t nrq = make_rsrc(nqb, span_bytes(nsq, p.q_rs));
            const i32x4 nrk = make_rsrc_words(nkb, span_bytes(nsk, p.k_rs));
            nrv = make_rsrc_words(nvb, span_bytes(nsk, p.v_rs));
            const int nmq = nm0 + wave * 32 + l32;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks)
                qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(nrq, (uint32_t)(nmq * p.q_rs + ks * 32 + hi * 16)));
#pragma unroll
            for (int i = 0; i < kDmaPerTile; ++i) dma1(nrk, p.k_rs, dk, kst + 0 * kTile, 0, i);
#pragma unroll
            for (int i = 0; i < kDmaPerTile; ++i) dma1(nrk, p.k_rs, dk, kst + 1 * kTile, 1, i);
#pragma unroll
            for (int i = 0; i < kDmaPerTile; ++i) dma1(nrv, p.v_rs, dv, vst + 0 * kTile, 0, i);
#pragma unroll
            for (int i = 0; i < kDmaPerTile; ++i) dma1(nrk, p.k_rs, dk, kst + 2 * kTile, 2, i);
#pragma unroll
            for (int i = 0; i < kDmaPerTile; ++i) dma1(nrv, p.v_rs, dv, vst + 1 * kTile, 1, i);
#pragma unroll
            for (int i = 0; i < kDmaPerTile; ++i) dma1(nrk, p.k_rs, dk, kst + 3 * kTile, 3, i);
            pref = true;
        }
    };
    // kTail: the last two steps of the launch (U = 2, 3 of its last group).
    // Their QK^T tiles (nsteps, nsteps + 1) and DMA tiles lie past the end,
    // so they run PV alone, with the softmax of tile nsteps - 1 in step 2.
    auto step = [&](auto u, int jj, auto tail_c) __attribute__((always_inline)) {
        constexpr int U = decltype(u)::value;
        constexpr bool kTail = decltype(tail_c)::value;
        static_assert(!kTail || U >= 2, "only the last two steps of a group skip QK^T");
        // Iteration jj loads K tile jj+5 and V tile jj+3. The wide forms
        // rebase the K resource at that tile every iteration (scalar work
        // only), so each K load takes its lane offset as it is, and move a
        // token-major V window on at the first iteration of every group of
        // four (its loads, tiles jj+3 .. jj+6, stay inside the window). The
        // d-major V resource is never rebased.
        if constexpr (kWide && !kTail) rk = window(kb, p.k_rs, jj + 5);
        if constexpr (kWide && !kVT && U == 0) {
            if (jj > 0) advance(rv, p.v_rs, jj);
        }
        const int kt = kWide ? 0 : jj + 5;
        const int vt = kWide && !kVT ? U + 3 : jj + 3;
        // The four loads are spread over the iteration so that their LDS
        // writes do not arrive as one burst that holds up the fragment reads.
        auto hook = [&](int k) __attribute__((always_inline)) {
            if (k == 0) dma_k1(kt, (U + 1) & 3, 0);
            if (k == 8) dma_k1(kt, (U + 1) & 3, 1);
            if (k == 16) dma_v1(vt, (U + 3) & 3, 0);
            if (k == 24) dma_v1(vt, (U + 3) & 3, 1);
        };
        if constexpr (kTail) {
            constexpr std::integral_constant<int, U == 2 ? 1 : 0> sm{};
            if constexpr (kPersist && U == 2) prefetch();
            if constexpr (kPersist && U == 3) {
                if (pref) {
#pragma unroll
                    for (int i = 0; i < kDmaPerTile; ++i) dma1(nrv, p.v_rs, dv, vst + 2 * kTile, 2, i);
                }
            }
            if constexpr (U & 1)
                iterate(std::false_type{}, sm, std::true_type{}, 0, U, jj + 1, sa, sb, pfb, pfa, -1, no_hook);
            else
                iterate(std::false_type{}, sm, std::true_type{}, 0, U, jj + 1, sb, sa, pfa, pfb, -1, no_hook);
        } else if constexpr (U & 1) {
            iterate(std::true_type{}, kSoftmax, std::true_type{}, (U + 2) & 3, U, jj + 1, sa, sb, pfb, pfa,
                    (U + 3) & 3, hook);
        } else {
            iterate(std::true_type{}, kSoftmax, std::true_type{}, (U + 2) & 3, U, jj + 1, sb, sa, pfa, pfb,
                    (U + 3) & 3, hook);
        }
        // The tail steps issue none of this tile's loads (and a persistent
        // launch's prefetch must stay in flight).
        if constexpr (!(kPersist && kTail)) wait_vmcnt<2 * kDmaPerTile>();
        barrier();
    };
    int j = 0;
    for (; j < nsteps - 4; j += 4) {
        step(std::integral_constant<int, 0>{}, j, std::false_type{});
        step(std::integral_constant<int, 1>{}, j + 1, std::false_type{});
        step(std::integral_constant<int, 2>{}, j + 2, std::false_type{});
        step(std::integral_constant<int, 3>{}, j + 3, std::false_type{});
    }
    if constexpr (kWide) {
        // Take the lane again for the last steps and the epilogue rather
        // than hold it across the key loop.
        lane = lane_from_hw();
        hi = lane >> 5;
        l32 = lane & 31;
    }
    if (nsteps > 0) {
        step(std::integral_constant<int, 0>{}, j, std::false_type{});
        step(std::integral_constant<int, 1>{}, j + 1, std::false_type{});
        step(std::integral_constant<int, 2>{}, j + 2, std::true_type{});
        step(std::integral_constant<int, 3>{}, j + 3, std::true_type{});
    }
    if (!pref) wait_vmcnt<0>();  // no LDS DMA may still land after the workgroup ends (a prefetch lands for the next tile)

    // Epilogue: combine the two halves' partial sums, normalise, store.
    {
        f32x2 pr = halves(l_run);
        l_run = pr.x + pr.y;
    }
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    const float lse = l_run > 0.f ? (mc + __log2f(l_run)) * 0.69314718055994531f : -INFINITY;
    // Query row of the lane: the wide forms take it from the lane taken
    // after the key loop rather than hold it across the loop.
    const int emq = kWide ? m0 + wave * 32 + l32 : mq;
    // This wave's 32 rows of O, normalised to bf16, written through its
    // 2 KB of V stage 3. The stage is free here: its last reader, the final
    // step's PV, finished before that step's barrier; a persistent launch's
    // prefetch fills the other stages; a later call writes it only in its
    // first main-loop step, and there each wave's DMA fills exactly its own
    // 2 KB (eight 256-byte key rows, or sixteen 128-byte dim rows of a
    // d-major tile) after its own reads here. A lane holds four dims of
    // every 8-dim block of one row; in four passes of 32 dims the lanes
    // write their pieces, then each reads back 16 bytes, four lanes one
    // row's 64 contiguous bytes, and stores them: 128 L2 requests per wave
    // instead of 512 for 8-byte stores straight from the accumulators
    // (short tiles ran up to 15% faster). One wave's LDS accesses run in
    // order, so each pass reads what it wrote and the next writes over what
    // was read. 16-byte chunks are XOR-swizzled by row pair: the reads are
    // bank-conflict free. Row r of the wave goes to base + r * row_bytes
    // when r < rows.
    auto staged_store = [&](char* base, int64_t row_bytes, int rows) __attribute__((always_inline)) {
        typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
        typedef __attribute__((address_space(3))) i32x4 lds_i32x4;
        lds_char* const staged = (lds_char*)(vst + 3 * kTile) + wave * 32 * 64;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                i32x2 w;
                w.x = (int)pack_bf16x2(oacc[db][i * 4 + 0] * inv, oacc[db][i * 4 + 1] * inv);
                w.y = (int)pack_bf16x2(oacc[db][i * 4 + 2] * inv, oacc[db][i * 4 + 3] * inv);
                *(lds_i32x2*)(staged + l32 * 64 + (((i ^ ((l32 >> 1) & 3)) << 4) | (hi << 3))) = w;
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int row = (lane >> 2) + 16 * k, c = lane & 3;
                const i32x4 v = *(const lds_i32x4*)(staged + row * 64 + ((c ^ ((row >> 1) & 3)) << 4));
                if (row < rows) *(i32x4*)(base + (int64_t)row * row_bytes + db * 64 + c * 16) = v;
            }
        }
    };
    if (slot >= 0) {
        // Partial result of a key-range piece: normalised O in bf16 (as the
        // output itself is rounded) and the LSE in fp32, every row.
        staged_store((char*)(p.ws_o + ((int64_t)slot * kBM + wave * 32) * kD), kD * 2, 32);
        if (hi == 0) p.ws_lse[(int64_t)slot * kBM + wave * 32 + l32] = lse;
        return false;
    }
    const int wrow = m0 + wave * 32;  // the wave's first query row
    staged_store((char*)p.o + 2 * (b * p.o_sb + h * p.o_sh) + (int64_t)(q0 + wrow) * p.o_rs, p.o_rs, sq - wrow);
    if (emq < sq && p.lse != nullptr && hi == 0) p.lse[b * p.lse_sb + h * p.lse_sh + q0 + emq] = lse;
    return pref;
}

// The dynamic tail: the last round's tiles are cut into key-range pieces
// that the workgroups after the whole tiles take from a counter in the
// workspace as they free up, so CUs that ran their whole tiles faster (XCD
// clocks differ) take more of the tail.
template <bool kWide, bool kVT>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(AttnParams p) {
    __shared__ int queue_head;
    // Workgroups are dispatched round-robin over the 8 XCDs, workgroup i to
    // XCD i % 8 as its (i / 8)-th. Dense grids are renumbered so that each
    // XCD runs one contiguous range of tiles: its 32 resident workgroups are
    // then consecutive query tiles of one head and stream that head's K/V
    // through the XCD's L2 once per round (0.98 GB of HBM reads per launch at
    // B=1 H=5 S=49,920; 1.70 GB in dispatch order, at the same speed). A
    // static split (fewer tiles than CUs, n_full == 0) gives every workgroup
    // one piece, each XCD a contiguous range of them.
    // Packed varlen launches with a work list (vplan) run the list's whole
    // rounds in dispatch order and take the last round's pieces from a
    // counter. Without a list they keep dispatch order too (tile i is
    // workgroup i): tiles past a short segment's end exit at once, and in
    // dispatch order they spread over all XCDs (contiguous ranges gave a few
    // XCDs nearly only empty tiles: the 49,920 + 1,296 two-segment batch ran
    // at half speed).
    const int bid = blockIdx.x;
    // First work item of this wave (wide forms: read once, kept as a scalar).
    const int wave_first = kWide ? __builtin_amdgcn_readfirstlane((int)threadIdx.x) & ~63 : 0;
    int tile = bid, chunk = -1, chunks = 1, slot = -1;
    const bool planned = p.vplan != nullptr;
    // With a tail queue, the workgroups after the whole tiles take the pieces
    // of the last round's tiles from a counter, one at a time.
    const bool queued = planned ? bid >= p.ub_tiles : p.queue != nullptr && bid >= p.n_full;
    if (planned && !queued) {
        // Dispatch order over the list: its tiles differ in length (longest
        // first), and round-robin over the XCDs gives every XCD an even share
        // of each length (XCD-contiguous ranges gave XCD 0 all the longest).
        if (bid >= p.vplan[kPlanFull]) return;
        tile = __builtin_amdgcn_readfirstlane(p.vlist[bid]);  // uniform: the addressing is scalar
    } else if (p.cu_q == nullptr && !queued) {
        const int nb = p.queue != nullptr ? p.n_full : (int)gridDim.x;
        const int xcd = bid & 7, local = bid >> 3, per = nb >> 3, rem = nb & 7;
        const int start = xcd * per + min(xcd, rem);  // first tile of this XCD's share
        tile = start + local;
        if (p.split_n != 0) {
            const int full_per = p.n_full >> 3;  // n_full: 0, or whole rounds of CUs (a multiple of 8)
            if (local < full_per) {
                tile = xcd * full_per + local;
            } else {
                slot = start - xcd * full_per + (local - full_per);
                tile = p.n_full + slot % p.split_tiles;
                chunk = slot / p.split_tiles;
                chunks = p.split_n;
            }
        }
    }
    // Two call sites: the whole tiles keep a straight-line copy of the tile
    // code (a single call inside the loop below changed its register
    // allocation and made it 1-2% slower).
    if (!queued) {
        attn_tile<kWide, kVT>(p, tile, chunk, chunks, slot, false, nullptr, false, -1, nullptr, nullptr, wave_first);
        return;
    }
    int* const counter = planned ? (int*)p.vplan + kPlanQueue : p.queue;
    // The wide forms find the first work item from wave_first and the lane,
    // so no VGPR holds the id across the loop.
    const bool leader = kWide ? wave_first + lane_from_hw() == 0 : threadIdx.x == 0;
    for (;;) {
        if (leader) queue_head = atomicAdd(counter, 1);
        __syncthreads();  // also: every wave is done with the previous piece's LDS
        const int piece = __builtin_amdgcn_readfirstlane(queue_head);  // uniform: keep it scalar
        __syncthreads();  // every wave has read queue_head before it is written again
        if (planned) {
            if (piece >= p.vplan[kPlanPieces]) return;
            // pieces[i] = (list position, chunk | chunks << 2 | (merge slot + 1) << 5)
            const int pos = __builtin_amdgcn_readfirstlane(p.vpieces[2 * piece]);
            const int code = __builtin_amdgcn_readfirstlane(p.vpieces[2 * piece + 1]);
            const int merge_slot = (code >> 5) - 1;
            tile = __builtin_amdgcn_readfirstlane(p.vlist[pos]);
            chunk = code & 3;
            chunks = (code >> 2) & 7;
            slot = merge_slot >= 0 ? merge_slot * kQueuePieces + chunk : -1;
        } else {
            if ((unsigned)piece >= (unsigned)(p.split_n * p.split_tiles)) return;
            tile = p.n_full + piece % p.split_tiles;
            chunk = piece / p.split_tiles;  // chunk-major: every tile's first pieces first
            chunks = p.split_n;
            slot = piece;
        }
        // The launch arguments are read afresh for each piece (an opaque zero
        // offset keeps the compiler from hoisting the loads), from the
        // kernel-argument segment through the scalar cache, rather than held
        // in scalar registers across the loop: the piece's own addressing
        // needs those registers (spills of scalar registers to VGPR lanes
        // fell from 84 to 28 in the dense kernel).
        int zero;
        asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
        KernArgs* pk = (KernArgs*)((const __attribute__((address_space(4))) char*)&p + zero);
        attn_tile<kWide, kVT>(*pk, tile, chunk, chunks, slot, !planned, nullptr, false, -1, nullptr, nullptr, wave_first);
    }
}

// The work list of a packed varlen launch, built on the device from the
// segment offsets (the host does not have them) by one 256-thread workgroup:
//   1. the query and key length of every segment (clamped as attn_tile
//      clamps them);
//   2. segments ordered by key length, longest first (ties: segment order;
//      up to kPlanSortMax segments, beyond that in segment order), so the
//      longest tiles run first and the last round holds the shortest;
//   3. the non-empty (segment, head, query tile) tiles in that order, the
//      heads and query tiles of one segment consecutive (they share K/V);
//   4. n_full = the whole rounds but the last (as for dense launches), and
//      the last round's tiles cut into key-range pieces (kQueuePieces, fewer
//      when a piece would hold under kQueueMinKeyTiles key tiles; one piece
//      writes the output itself), with merge slots for the split tiles;
//   5. the counts, and the tail counter zeroed.
constexpr int kPlanSortMax = 2048;

// Exclusive prefix sum over the 256 threads; *total receives the sum.
__device__ __forceinline__ int block_scan(int v, int* buf, int* total) {
    const int t = threadIdx.x;
    buf[t] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const int add = t >= off ? buf[t - off] : 0;
        __syncthreads();
        buf[t] += add;
        __syncthreads();
    }
    const int incl = buf[t];
    *total = buf[255];
    __syncthreads();
    return incl - v;
}

// Packed launches of short segments without a work list: one workgroup per CU
// runs tile after tile, and each tile issues the next one's Q loads and first
// K / V DMA during its own last two iterations, so the next tile starts with
// them in flight or landed instead of paying their latency (5-7 us against
// 1.5 us per key tile). Tiles [0, grid) start one per workgroup; every later
// one is claimed from the counter at p.persist_queue (tile grid + claim),
// two tiles ahead of its run, so the claim's latency passes during a tile and
// workgroups that drew short tiles take more of them.
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_persist_kernel(AttnParams p) {
    __shared__ int claim;
    const int total = p.n_qtiles * p.heads * p.n_groups;
    const int grid = (int)gridDim.x;
    // Segment bounds of tile t, loaded one tile ahead: they have landed when
    // the tile starts, and the next tile's by the time its loads are issued.
    // Read through the constant address space (nothing writes them during
    // the launch): scalar loads, which vector-memory waits do not count.
    using ConstInt = const __attribute__((address_space(4))) int;
    ConstInt* const cq = (ConstInt*)(uintptr_t)p.cu_q;
    ConstInt* const ck = (ConstInt*)(uintptr_t)p.cu_k;
    auto bounds = [&](int t, int* c) {
        const int s = t / p.n_qtiles / p.heads;
        c[0] = cq[s];
        c[1] = cq[s + 1];
        c[2] = ck[s];
        c[3] = ck[s + 1];
    };
    // Every wave reads the claim before thread 0 writes the next one.
    auto broadcast = [&](int c) {
        if (threadIdx.x == 0) claim = c;
        __syncthreads();
        const int v = __builtin_amdgcn_readfirstlane(claim);
        __syncthreads();
        return grid + v < total ? grid + v : -1;
    };
    int t = blockIdx.x;  // grid <= total
    int nt = broadcast(threadIdx.x == 0 ? atomicAdd(p.persist_queue, 1) : 0);
    bf16x8 qf[8];
    int cur[4], nxt[4];
    bool pre = false;
    bounds(t, cur);
    for (;;) {
        bounds(nt >= 0 ? nt : t, nxt);
        int c_after = 0;
        if (nt >= 0 && threadIdx.x == 0) c_after = atomicAdd(p.persist_queue, 1);
        // The arguments through an opaque address, as in the tail loop above.
        int zero;
        asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
        KernArgs* pk = (KernArgs*)((const __attribute__((address_space(4))) char*)&p + zero);
        pre = attn_tile<false, false, true>(*pk, t, -1, 1, -1, false, qf, pre, nt, cur, nxt);
        if (nt < 0) break;
        t = nt;
        nt = broadcast(c_after);
#pragma unroll
        for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
    }
}

__global__ __launch_bounds__(256) void attn_varlen_plan_kernel(AttnParams p) {
    __shared__ int scan[256];
    // Per-segment arrays: in LDS up to kPlanSortMax segments (the planner is
    // a chain of dependent accesses, so their latency is its time), in the
    // workspace beyond.
    __shared__ int lds_seg[4 * kPlanSortMax];
    const int t = threadIdx.x;
    const int nseg = p.n_groups, heads = p.heads, nq = p.n_qtiles, cus = p.plan_cus;
    int* const info = p.vplan_w;
    int* const list = p.vlist_w;
    int* const pieces = p.vpieces_w;
    int* const merge = p.vmerge_w;
    const bool sorted = nseg <= kPlanSortMax;
    int* const segq = sorted ? lds_seg : p.vscratch;
    int* const segk = segq + nseg;
    int* const order = segk + nseg;
    int* const base = order + nseg;
    for (int i = t; i < nseg; i += 256) {
        const int q0 = min(max(p.cu_q[i], 0), p.seqlen_q);
        const int k0 = min(max(p.cu_k[i], 0), p.seqlen_k);
        segq[i] = min(max(p.cu_q[i + 1], q0), p.seqlen_q) - q0;
        segk[i] = min(max(p.cu_k[i + 1], k0), p.seqlen_k) - k0;
    }
    __syncthreads();
    for (int i = t; i < nseg; i += 256) {
        int r = i;
        if (sorted) {
            const int li = segk[i];
            r = 0;
            for (int j = 0; j < nseg; ++j) r += (segk[j] > li) | ((segk[j] == li) & (j < i));
        }
        order[r] = i;
    }
    __syncthreads();
    // Tiles of the segments in that order (query rows past n_qtiles tiles
    // are not computed: max_seqlen_q bounds every segment).
    int carry = 0;
    for (int c0 = 0; c0 < nseg; c0 += 256) {
        const int r = c0 + t;
        const int cnt = r < nseg ? min((segq[order[r]] + kBM - 1) / kBM, nq) * heads : 0;
        int tot;
        const int off = block_scan(cnt, scan, &tot);
        if (r < nseg) base[r] = carry + off;
        carry += tot;
    }
    // Offsets that ascend give at most ub_tiles tiles; others are cut there.
    const int n_tiles = min(carry, p.ub_tiles);
    __syncthreads();
    for (int r = 0; r < nseg; ++r) {
        const int seg = order[r];
        const int tq = min((segq[seg] + kBM - 1) / kBM, nq);
        const int b0 = base[r];
        for (int u = t; u < tq * heads && b0 + u < n_tiles; u += 256) list[b0 + u] = (seg * heads + u / tq) * nq + u % tq;
    }
    const int n_full = n_tiles > cus ? (n_tiles - 1) / cus * cus : 0;
    const int n_last = n_tiles - n_full;
    int piece_carry = 0, merge_carry = 0;
    for (int c0 = 0; c0 < n_last; c0 += 256) {
        const int i = c0 + t;
        int n = 0;
        if (i < n_last) {
            // Segment of list position n_full + i: the last r with base[r] <=
            // the position (empty segments share their successor's base).
            const int pos = n_full + i;
            int lo = 0, hi = nseg - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (base[mid] <= pos) lo = mid; else hi = mid - 1;
            }
            const int nkt = (segk[order[lo]] + kBN - 1) / kBN;
            n = kQueuePieces;
            while (n > 1 && nkt / n < kQueueMinKeyTiles) --n;
        }
        int ptot, mtot;
        const int poff = block_scan(n, scan, &ptot);
        const int moff = block_scan(n > 1 ? 1 : 0, scan, &mtot);
        if (i < n_last) {
            const int pos = n_full + i;
            const int ms = n > 1 ? merge_carry + moff : -1;
            for (int c = 0; c < n; ++c) {
                pieces[2 * (piece_carry + poff + c)] = pos;
                pieces[2 * (piece_carry + poff + c) + 1] = c | (n << 2) | ((ms + 1) << 5);
            }
            if (ms >= 0) {
                merge[2 * ms] = pos;
                merge[2 * ms + 1] = n;
            }
        }
        piece_carry += ptot;
        merge_carry += mtot;
    }
    if (t == 0) {
        info[kPlanTiles] = n_tiles;
        info[kPlanFull] = n_full;
        info[kPlanPieces] = piece_carry;
        info[kPlanMerges] = merge_carry;
        info[kPlanQueue] = 0;
    }
}

// d-major copy of V for the kVT form: vt holds, per (batch, head), 128 rows
// (head dims) of vt_rs bytes with keys contiguous, zero from seqlen_k to the
// next multiple of kBN. One workgroup moves a 64-key x 128-dim block through
// LDS: 16-byte row loads in, 16-byte dim-row stores out (8 lanes per 128-byte
// row). Rows are 65 dwords in LDS, so both phases are bank-conflict free.
__global__ __launch_bounds__(256) void attn_vt_kernel(AttnParams p) {
    __shared__ uint32_t blk[kBN * 65];
    const int t = threadIdx.x;
    const int h = blockIdx.y, b = blockIdx.z;
    // The dynamic tail's counter, for the attention kernel that follows on
    // the stream (instead of a launch of attn_queue_reset).
    if (p.queue != nullptr && t == 0 && blockIdx.x == 0 && h == 0 && b == 0) *p.queue = 0;
    // Block x moves keys [64x, 64x + 64) of the d-major layout. Dense: key k
    // of the sequence sits at k. Packed varlen: segment s starts at
    // vt_segment_start (its own rows, padded to a multiple of 64).
    const int k0 = blockIdx.x * kBN;
    int src0 = k0, src_end = p.seqlen_k;
    if (p.cu_k != nullptr) {
        // The grid covers every key of the rows; keys outside every segment
        // (padding, gaps) are written as zeros, so the attention kernel never
        // reads uninitialised memory past a segment's end.
        const int nseg = p.n_groups;
        int lo = 0, hi = nseg - 1;  // the last segment starting at or before k0
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (vt_segment_start(min(max(p.cu_k[mid], 0), p.seqlen_k), mid) <= k0) lo = mid; else hi = mid - 1;
        }
        const int s0 = min(max(p.cu_k[lo], 0), p.seqlen_k);
        const int s1 = min(max(p.cu_k[lo + 1], s0), p.seqlen_k);
        const int v0 = vt_segment_start(s0, lo);
        src0 = s0 + (k0 - v0);
        src_end = k0 >= v0 ? s1 : src0;  // before the first segment's start: zeros
    }
    const char* src = (const char*)p.v + 2 * (b * p.v_sb + h * p.v_sh);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int key = i * 16 + (t >> 4), c = t & 15;
        i32x4 x = i32x4{0, 0, 0, 0};
        if (src0 + key < src_end) x = *(const i32x4*)(src + (int64_t)(src0 + key) * p.v_rs + c * 16);
        uint32_t* row = blk + key * 65 + c * 4;
        row[0] = (uint32_t)x.x;
        row[1] = (uint32_t)x.y;
        row[2] = (uint32_t)x.z;
        row[3] = (uint32_t)x.w;
    }
    __syncthreads();
    char* dst = (char*)p.vt + 2 * (b * p.vt_sb + h * p.vt_sh + (int64_t)k0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = i * 32 + (t >> 3), kc = t & 7;
        const int sh = (d & 1) * 16;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = blk[(8 * kc + 2 * j) * 65 + (d >> 1)] >> sh;
            const uint32_t up = blk[(8 * kc + 2 * j + 1) * 65 + (d >> 1)] >> sh;
            w[j] = (lo & 0xffffu) | (up << 16);
        }
        *(i32x4*)(dst + (int64_t)d * p.vt_rs + kc * 16) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

// Zeroes the dynamic tail's counter (a kernel, not a memset, so that the
// launch can be captured in a graph).
__global__ void attn_queue_reset(int* queue) {
    if (threadIdx.x == 0) *queue = 0;
}

// Combines the split_n partial results of each split tile: with weights
// w_i = exp(lse_i - max lse), O = sum w_i O_i / sum w_i and
// LSE = max lse + log(sum w_i). 32 rows per workgroup, 8 lanes per row,
// 16 head dims per lane. kMaxP >= split_n sizes the registers of the loaded
// rows (4 or 8); every LSE and row of the pieces is loaded in one unrolled
// sequence, ending on a wave-uniform branch at split_n, before any is used.
constexpr int kMergeRows = 32;

template <int kMaxP>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p) {
    const int split_tile = blockIdx.x / (kBM / kMergeRows);
    const int row = (blockIdx.x % (kBM / kMergeRows)) * kMergeRows + threadIdx.x / 8;
    const int d0 = (threadIdx.x % 8) * 16;
    // Dense: split tile i is tile n_full + i, its piece c in slot
    // c * split_tiles + i. Planned varlen: merge slot i names a list position
    // and its piece count (the grid is an upper bound), piece c in slot
    // i * kQueuePieces + c.
    int tile = p.n_full + split_tile, n = p.split_n;
    int64_t slot0 = split_tile, slot_step = p.split_tiles;
    if (p.vplan != nullptr) {
        if (split_tile >= p.vplan[kPlanMerges]) return;
        tile = p.vlist[p.vmerge[2 * split_tile]];
        n = p.vmerge[2 * split_tile + 1];
        slot0 = (int64_t)split_tile * kQueuePieces;
        slot_step = 1;
    }
    const int qt = tile % p.n_qtiles;
    const int rest = tile / p.n_qtiles;
    const int h = rest % p.heads;
    int b = rest / p.heads, q0 = 0, sq = p.seqlen_q;
    if (p.cu_q != nullptr) {
        q0 = min(max(p.cu_q[b], 0), p.seqlen_q);
        sq = min(max(p.cu_q[b + 1], q0), p.seqlen_q) - q0;
        b = 0;
    }
    const int mq = qt * kBM + row;
    if (mq >= sq) return;
    float lq[kMaxP];
    i32x4 part[kMaxP][2];  // 16 bf16 head dims of the row per piece
#pragma unroll
    for (int c = 0; c < kMaxP; ++c) {
        if (c >= n) break;
        const int64_t pc = slot0 + c * slot_step;
        lq[c] = p.ws_lse[pc * kBM + row];
        const i32x4* src = (const i32x4*)(p.ws_o + (pc * kBM + row) * kD + d0);
        part[c][0] = src[0];
        part[c][1] = src[1];
    }
    float lse_max = -INFINITY;
#pragma unroll
    for (int c = 0; c < kMaxP; ++c) {
        if (c >= n) break;
        lse_max = fmaxf(lse_max, lq[c]);
    }
    f32x4 acc[4] = {f32x4{}, f32x4{}, f32x4{}, f32x4{}};
    float wsum = 0.f;
#pragma unroll
    for (int c = 0; c < kMaxP; ++c) {
        if (c >= n) break;
        // Every piece holds keys and writes all its rows; a -inf LSE would
        // still weigh nothing.
        const float w = lq[c] == -INFINITY ? 0.f : __expf(lq[c] - lse_max);
        wsum += w;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (uint32_t)part[c][i >> 1][2 * (i & 1)], up = (uint32_t)part[c][i >> 1][2 * (i & 1) + 1];
            const f32x4 x{__uint_as_float(lo << 16), __uint_as_float(lo & 0xffff0000u), __uint_as_float(up << 16),
                          __uint_as_float(up & 0xffff0000u)};
            acc[i] += w * x;
        }
    }
    const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
    char* ob = (char*)p.o + 2 * (b * p.o_sb + h * p.o_sh + d0) + (int64_t)(q0 + mq) * p.o_rs;
    i32x4 w0, w1;
    w0.x = (int)pack_bf16x2(acc[0].x * inv, acc[0].y * inv);
    w0.y = (int)pack_bf16x2(acc[0].z * inv, acc[0].w * inv);
    w0.z = (int)pack_bf16x2(acc[1].x * inv, acc[1].y * inv);
    w0.w = (int)pack_bf16x2(acc[1].z * inv, acc[1].w * inv);
    w1.x = (int)pack_bf16x2(acc[2].x * inv, acc[2].y * inv);
    w1.y = (int)pack_bf16x2(acc[2].z * inv, acc[2].w * inv);
    w1.z = (int)pack_bf16x2(acc[3].x * inv, acc[3].y * inv);
    w1.w = (int)pack_bf16x2(acc[3].z * inv, acc[3].w * inv);
    *(i32x4*)ob = w0;
    *(i32x4*)(ob + 16) = w1;
    if (p.lse != nullptr && d0 == 0)
        p.lse[b * p.lse_sb + h * p.lse_sh + q0 + mq] = wsum > 0.f ? lse_max + __logf(wsum) : -INFINITY;
}

}  // namespace

int attn_fwd_block_m() { return kBM; }
int attn_fwd_persist_max_rows() { return kPersistMaxQTiles * kBM; }
int attn_fwd_tail_pieces() { return kQueuePieces; }
int64_t attn_fwd_piece_bytes() { return (int64_t)kBM * (kD * 2 + 4); }
int attn_fwd_block_n() { return kBN; }
int attn_fwd_window_rows() { return kWindowRows > kBM ? kWindowRows : kBM; }
int attn_fwd_row_margin() { return kBM + kBN * (2 * kStages + 2); }

SplitPlan plan_attn_split(int64_t tiles, int64_t key_tiles, int cus, int64_t max_workspace) {
    SplitPlan plan{(int32_t)tiles, 0, 0, 0, 0, 0};
    if (cus < 8 || cus % 8 != 0 || tiles <= 0) return plan;
    const int64_t piece_bytes = attn_fwd_piece_bytes();  // bf16 partial O and fp32 LSE of a piece's rows
    if (tiles > cus) {
        // Dynamic tail: the whole rounds but the last run as they are; the
        // last round's tiles become kQueuePieces key-range pieces each, taken
        // from a counter by cus workgroups (at most) as CUs free up. Pieces
        // keep at least kQueueMinKeyTiles key tiles, so the pipeline's fill
        // and drain stay small against a piece; fewer pieces are cut when
        // their partial results would not fit in max_workspace.
        const int64_t full = (tiles - 1) / cus * cus, rest = tiles - full;
        auto bytes = [&](int n) { return ((int64_t)n * rest * piece_bytes + 255) / 256 * 256 + 256; };
        int n = kQueuePieces;
        while (n > 1 && (key_tiles / n < kQueueMinKeyTiles || bytes(n) > max_workspace)) --n;
        if (n < 2) return plan;
        plan.n_full = (int32_t)full;
        plan.split_n = n;
        plan.split_tiles = (int32_t)rest;
        plan.queue_blocks = (int32_t)(rest * n < cus ? rest * n : cus);
        plan.queue_offset = ((int64_t)n * rest * piece_bytes + 255) / 256 * 256;
        plan.workspace_bytes = bytes(n);
        return plan;
    }
    // One partial round: its tiles are cut into n key-range pieces when that
    // shortens the round (n <= 8, at least one key tile per piece):
    // ceil(tiles * n / cus) / n. The chip is power-bound under this kernel:
    // a round that keeps 70% or more of the CUs busy runs at a higher clock
    // and loses little, and splitting it does not pay for the pieces and the
    // merge.
    if (tiles * 10 >= (int64_t)cus * 7) return plan;
    double best = 1.0;
    int best_n = 0;
    for (int n = 2; n <= 8 && n <= key_tiles; ++n) {
        if ((int64_t)n * tiles * piece_bytes > max_workspace) break;
        const double cost = (double)((tiles * n + cus - 1) / cus) / n;
        if (cost < best - 0.05) {
            best = cost;
            best_n = n;
        }
    }
    if (best_n == 0) return plan;
    plan.n_full = 0;
    plan.split_n = best_n;
    plan.split_tiles = (int32_t)tiles;
    plan.workspace_bytes = (int64_t)best_n * tiles * piece_bytes;
    return plan;
}

hipError_t attn_static_scratch(void** ptr) {
    // Looked up once per device (with that device current), then cached.
    static std::atomic<void*> cache[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev >= 0 && dev < 64) {
        void* hit = cache[dev].load(std::memory_order_acquire);
        if (hit != nullptr) {
            *ptr = hit;
            return hipSuccess;
        }
    }
    void* addr = nullptr;
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (dev >= 0 && dev < 64) cache[dev].store(addr, std::memory_order_release);
    *ptr = addr;
    return hipSuccess;
}

hipError_t launch_attn_fwd(const AttnParams& p, hipStream_t stream) {
    const int64_t tiles = (int64_t)p.n_qtiles * p.heads * p.n_groups;
    if (tiles <= 0) return hipSuccess;
    int64_t blocks = tiles;
    if (p.vplan != nullptr) {
        // The list, its pieces and the d-major V offsets first.
        hipLaunchKernelGGL(attn_varlen_plan_kernel, dim3(1), dim3(256), 0, stream, p);
        blocks = (int64_t)p.ub_tiles + p.plan_cus;
    } else if (p.queue != nullptr) {
        // With a d-major V copy the transpose kernel zeroes the counter.
        if (p.vt == nullptr) hipLaunchKernelGGL(attn_queue_reset, dim3(1), dim3(64), 0, stream, p.queue);
        blocks = (int64_t)p.n_full + p.queue_blocks;
    } else if (p.split_n != 0) {
        blocks = (int64_t)p.n_full + (int64_t)p.split_n * p.split_tiles;
    }
    if (p.vt != nullptr) {
        // Dense: the keys of the sequence; varlen: every key of the padded rows.
        const int64_t vt_tiles = (p.seqlen_k + kBN - 1) / kBN + (p.cu_k != nullptr ? p.n_groups : 0);
        const dim3 tgrid((unsigned)vt_tiles, (unsigned)p.heads, (unsigned)(p.cu_k != nullptr ? 1 : p.n_groups));
        hipLaunchKernelGGL(attn_vt_kernel, tgrid, dim3(256), 0, stream, p);
    }
    const dim3 block(kThreads);
    // Persistent only for short segments (at most kPersistMaxQTiles query
    // tiles each), where a tile's fixed cost is a large share of it.
    if (p.cu_q != nullptr && p.vplan == nullptr && !p.wide && p.vt == nullptr && p.split_n == 0 &&
        p.queue == nullptr && p.persist_queue != nullptr && p.persist_blocks > 0 && p.n_qtiles <= kPersistMaxQTiles) {
        const int64_t n = blocks < p.persist_blocks ? blocks : p.persist_blocks;
        hipLaunchKernelGGL(attn_queue_reset, dim3(1), dim3(64), 0, stream, p.persist_queue);
        hipLaunchKernelGGL(attn_fwd_persist_kernel, dim3((unsigned)n), block, 0, stream, p);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)blocks);
    if (p.wide && p.vt != nullptr)
        hipLaunchKernelGGL((attn_fwd_kernel<true, true>), grid, block, 0, stream, p);
    else if (p.wide)
        hipLaunchKernelGGL((attn_fwd_kernel<true, false>), grid, block, 0, stream, p);
    else if (p.vt != nullptr)
        hipLaunchKernelGGL((attn_fwd_kernel<false, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<false, false>), grid, block, 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.vplan != nullptr) {
        // Every possible merge slot (at most plan_cus split tiles); slots past
        // the plan's count exit.
        const dim3 merge_grid((unsigned)(p.plan_cus * (kBM / kMergeRows)));
        hipLaunchKernelGGL(attn_merge_kernel<4>, merge_grid, dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    if (p.split_n == 0) return e;
    const dim3 merge_grid((unsigned)(p.split_tiles * (kBM / kMergeRows)));
    if (p.split_n <= 4)
        hipLaunchKernelGGL(attn_merge_kernel<4>, merge_grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(attn_merge_kernel<8>, merge_grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace h3a
