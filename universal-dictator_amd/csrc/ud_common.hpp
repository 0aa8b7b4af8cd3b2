// Shared device helpers for the gfx950 encoder-step kernels: bf16 and IEEE-half storage, wave64
// reductions, vector loads, activations.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace ud {

typedef uint16_t bf16;  // bfloat16 storage (upper half of an fp32)

// Widening is a shift (Sources/DictatorEngine/Metal/00_common.metal:32).
__device__ __forceinline__ float bf2f(bf16 b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even, NaN -> 0x7FC0 (Sources/DictatorEngine/Core/Tensor.swift:116-122).
__device__ __forceinline__ bf16 f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
    return (bf16)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// MFMA operand types (v_mfma_f32_16x16x32_bf16: 8 bf16 of A and of B per lane, 4 fp32 of C).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
// Two floats rounded to nearest-even bf16 by v_cvt_pk_bf16_f32, packed (x in the low half).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
    const f32x2_t v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
    bf16x8_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}
// IEEE half operands (v_mfma_f32_16x16x32_f16) in the same fragment layout.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f16x8_t as_f16x8(uint4 v) {
    f16x8_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}
// fp32 -> IEEE half, round to nearest even, saturating: values beyond half's largest finite
// magnitude (65504, infinities included) are stored as +-65504, NaN stays NaN.  Every 16-bit
// activation, K/V cache row and table entry a 16-bit encoder writes goes through this, so a value
// that outgrows half's range is clipped instead of turning into inf (and NaN after the next
// LayerNorm).
constexpr float kHalfMaxF = 65504.0f;
__device__ __forceinline__ float sat_half_range(float f) {
    return __builtin_isnan(f) ? f : fminf(fmaxf(f, -kHalfMaxF), kHalfMaxF);
}
__device__ __forceinline__ _Float16 f2h_sat(float f) { return (_Float16)sat_half_range(f); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, f2h_sat(f)); }
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// A 16-bit operand value: IEEE half when H, bf16 otherwise (round to nearest even either way).
template <bool H> __device__ __forceinline__ uint16_t to16(float f) {
    if constexpr (H) return f2h(f);
    else return f2bf(f);
}

// Element types of the attention kernels: fp32, bf16 (uint16_t storage) and IEEE half (_Float16,
// the 16-bit format of a 16-bit encoder's activations, caches and tables).
typedef _Float16 f16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2_t as_half2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }
// The low / high half of a packed pair as fp32 (in an FMA, the conversion folds into v_fma_mix_f32).
__device__ __forceinline__ float half_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
__device__ __forceinline__ float half_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

template <typename T> __device__ __forceinline__ float to_f(T v);
template <> __device__ __forceinline__ float to_f<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f<bf16>(bf16 v) { return bf2f(v); }
template <> __device__ __forceinline__ float to_f<f16>(f16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f(float v);
template <> __device__ __forceinline__ float from_f<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float v) { return f2bf(v); }
template <> __device__ __forceinline__ f16 from_f<f16>(float v) { return f2h_sat(v); }

// SiLU x * sigmoid(x) (00_common.metal:25).
// SiLU and the logistic function with v_exp_f32 and v_rcp_f32 (about 1 ulp each) instead of an
// IEEE divide, whose correctly rounded sequence is ~10 instructions.  The reference's fp32
// x / (1 + exp(-x)) (Metal/00_common.metal:7-29) differs by a few ulp at most.  Limits:
// exp(-x) = inf gives 1 / inf = 0, so x -> -inf yields (-)0.
__device__ __forceinline__ float sigmoidf(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoidf(x); }

__device__ __forceinline__ float apply_act(float x, int act) {
    if (act == ACT_SILU) return silu(x);
    if (act == ACT_RELU) return x > 0.0f ? x : 0.0f;
    return x;
}

// 16-byte vector of storage elements: 8 bf16 or 4 fp32.
template <typename T> struct Vec16;
template <> struct Vec16<float> { static constexpr int N = 4; };
template <> struct Vec16<bf16> { static constexpr int N = 8; };
template <> struct Vec16<f16> { static constexpr int N = 8; };

// s_waitcnt immediate for "at most n vector-memory operations outstanding" (n < 64), every other
// counter left alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// Non-temporal 16-byte load: data read once per step (a stream's K/V window), streamed past the
// caches' normal retention.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
    const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// Unpack a 16-byte vector of T into floats (N = Vec16<T>::N values).
template <typename T> __device__ __forceinline__ void unpack16(uint4 v, float* f);
template <> __device__ __forceinline__ void unpack16<float>(uint4 v, float* f) {
    f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
}
template <> __device__ __forceinline__ void unpack16<bf16>(uint4 v, float* f) {
    f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xffff0000u);
    f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xffff0000u);
    f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xffff0000u);
    f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xffff0000u);
}
template <> __device__ __forceinline__ void unpack16<f16>(uint4 v, float* f) {
    f[0] = h2f((uint16_t)v.x); f[1] = h2f((uint16_t)(v.x >> 16));
    f[2] = h2f((uint16_t)v.y); f[3] = h2f((uint16_t)(v.y >> 16));
    f[4] = h2f((uint16_t)v.z); f[5] = h2f((uint16_t)(v.z >> 16));
    f[6] = h2f((uint16_t)v.w); f[7] = h2f((uint16_t)(v.w >> 16));
}

// DPP lane moves within 16-lane rows.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_1032 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// Cross-row sums with the gfx950 lane-swap instructions: a + (a from lane l^32) into lanes 0-31 and
// b + (b from lane l^32) into lanes 32-63; likewise for l^16 (rows 0, 2 get a, rows 1, 3 get b).
__device__ __forceinline__ float xsum32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Every lane receives op(v[l], v[l ^ 32]) (resp. v[l ^ 16]): the swap of v with itself hands each
// lane both values of its pair.
__device__ __forceinline__ float xmax32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xadd32(float v) { return xsum32(v, v); }
__device__ __forceinline__ float xadd16(float v) { return xsum16(v, v); }

// Sum over aligned groups of W lanes (W a power of two <= 64); every lane of a group receives the
// group total.  DPP inside a 16-lane row; the cross-row steps pair lane l with l ^ 16 and l ^ 32
// through the lane-swap instructions (VALU, no LDS round trip).
template <int W> __device__ __forceinline__ float group_sum(float v) {
    if constexpr (W >= 2) v += dpp_mov<DPP_QUAD_1032>(v);
    if constexpr (W >= 4) v += dpp_mov<DPP_QUAD_2301>(v);
    if constexpr (W >= 8) v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (W >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
    if constexpr (W >= 32) v = xadd16(v);
    if constexpr (W >= 64) v = xadd32(v);
    return v;
}

template <int W> __device__ __forceinline__ float group_max(float v) {
    if constexpr (W >= 2) v = fmaxf(v, dpp_mov<DPP_QUAD_1032>(v));
    if constexpr (W >= 4) v = fmaxf(v, dpp_mov<DPP_QUAD_2301>(v));
    if constexpr (W >= 8) v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
    if constexpr (W >= 16) v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
    if constexpr (W >= 32) v = xmax16(v);
    if constexpr (W >= 64) v = xmax32(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }



}  // namespace ud
