// Shared device helpers for the gfx950 kernels of the dense attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace h3a {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// Buffer resource word 3 for raw (stride 0) buffers on gfx9-family parts:
// 32-bit data format, offsets bounds-checked against num_records so that an
// out-of-range load returns 0 and an out-of-range store is dropped.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferWord3);
}

// The same resource as four words, for buffer instructions written as inline
// asm (the operand goes to an aligned SGPR quad).
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), (int)bytes, kBufferWord3};
}

__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

__device__ __forceinline__ void buf_store8(i32x2 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, 0);
}

// Value of `x` held by lane (lane ^ 32), combined with this lane's own value
// through `op`; v_permlane32_swap exchanges the two 32-lane halves of a wave.
__device__ __forceinline__ f32x2 halves(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    // lanes 0-31: r[0] = own, r[1] = lane+32; lanes 32-63: r[0] = lane-32, r[1] = own
    return f32x2{__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// DPP lane movement inside rows of 16 lanes (no LDS round trip, unlike
// ds_bpermute, which is what __shfl / __shfl_xor compile to).
enum : int {
    kDppXor1 = 0xB1,          // quad_perm [1,0,3,2]
    kDppXor2 = 0x4E,          // quad_perm [2,3,0,1]
    kDppHalfMirror = 0x141,   // lane i <- lane 7 - i within 8
    kDppMirror = 0x140,       // lane i <- lane 15 - i within 16
    kDppRor8 = 0x128,         // lane i <- lane (i + 8) mod 16, i.e. i ^ 8
};

template <int kCtrl>
__device__ __forceinline__ int dpp(int x) {
    return __builtin_amdgcn_update_dpp(0, x, kCtrl, 0xF, 0xF, false);
}

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(dpp<kCtrl>(__float_as_int(x)));
}

// Sum over aligned groups of L <= 16 lanes; every lane of a group receives
// the group's sum. Each step adds the partial sum of a disjoint set of lanes
// (pairs, quads, then mirrored halves), so all lanes must be active.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(L == 1 || L == 2 || L == 4 || L == 8 || L == 16, "group of at most 16 lanes");
    if constexpr (L >= 2) v += dpp<kDppXor1>(v);
    if constexpr (L >= 4) v += dpp<kDppXor2>(v);
    if constexpr (L >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (L >= 16) v += dpp<kDppMirror>(v);
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 b = __builtin_convertvector(f32x2{lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, b);
}

}  // namespace h3a
