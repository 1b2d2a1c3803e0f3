// kda_device.h -- device-side helpers shared by the KDA kernels (gfx950).
//
// bf16 storage is plain uint16_t: conversions are written out so the rounding
// (round-to-nearest-even, NaN kept quiet) is explicit and identical to torch's
// float -> bfloat16 cast. Cross-lane sums use DPP inside a 16-lane DPP row and
// one ds_swizzle for the 32-lane step; every lane of a group ends with the
// bitwise-identical sum (each step adds the same two partials, commuted).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kda {

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even (NaN stays a quiet NaN): the gfx950
// conversion instruction (v_cvt_pk_bf16_f32), same rounding as torch's cast.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two fp32 -> packed bf16 pair (lo in bits 0..15), one conversion instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Four consecutive elements of a bf16 or fp32 row, widened to fp32.
__device__ __forceinline__ float4 load4(const uint16_t *p) {
    const uint2 r = *reinterpret_cast<const uint2 *>(p);
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                       __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
}
__device__ __forceinline__ float4 load4(const float *p) {
    return *reinterpret_cast<const float4 *>(p);
}

typedef float kda_v4f __attribute__((ext_vector_type(4)));

// 16-byte streaming (nontemporal) access for data touched once per launch.
__device__ __forceinline__ float4 load4_stream(const float *p) {
    const kda_v4f t = __builtin_nontemporal_load(reinterpret_cast<const kda_v4f *>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void store4_stream(float *p, float4 v) {
    const kda_v4f t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<kda_v4f *>(p));
}

__device__ __forceinline__ float load1(const uint16_t *p) { return bf16_to_f32(*p); }
__device__ __forceinline__ float load1(const float *p) { return *p; }

__device__ __forceinline__ void store1(uint16_t *p, float x) { *p = f32_to_bf16(x); }
__device__ __forceinline__ void store1(float *p, float x) { *p = x; }

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// DPP controls (CDNA "DPP16" encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- 7-i within 8
constexpr int kDppRowMirror = 0x140;     // lane i <- 15-i within 16

// Sum over each aligned group of 16 lanes, result in every lane of the group.
__device__ __forceinline__ float group_sum16(float x) {
    x += dpp_mov<kDppQuadXor1>(x);
    x += dpp_mov<kDppQuadXor2>(x);
    x += dpp_mov<kDppRowHalfMirror>(x);
    x += dpp_mov<kDppRowMirror>(x);
    return x;
}

// Sum over each aligned group of 32 lanes.
__device__ __forceinline__ float group_sum32(float x) {
    x = group_sum16(x);
    // ds_swizzle bit mode: and_mask 0x1f, or_mask 0, xor_mask 0x10.
    x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
    return x;
}

template <int LANES>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(LANES == 16 || LANES == 32, "row groups are 16 or 32 lanes");
    if constexpr (LANES == 16) {
        return group_sum16(x);
    } else {
        return group_sum32(x);
    }
}

__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace kda
