// Shared helpers of the gfx950 kernels: vector types, error reporting and
// wave-level reductions. Every kernel in this library is written for wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/kunserve_hip.h"

namespace kunserve {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));  // fdot2 operand
typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors

void set_error(const char* fmt, ...);
void clear_error();

#define KSV_CHECK_ARG(cond, ...)              \
  do {                                        \
    if (!(cond)) {                            \
      ::kunserve::set_error(__VA_ARGS__);     \
      return KUNSERVE_EINVAL;                 \
    }                                         \
  } while (0)

#define KSV_CHECK_HIP(expr)                                                  \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess) {                                                  \
      ::kunserve::set_error("%s failed: %s", #expr, hipGetErrorString(_e)); \
      return KUNSERVE_EHIP;                                                  \
    }                                                                        \
  } while (0)

// Launch-error check right after a <<<>>> launch.
#define KSV_CHECK_LAUNCH() KSV_CHECK_HIP(hipGetLastError())

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Validates the pool descriptor for kernels that issue 16-byte loads along
// head_dim. Returns KUNSERVE_OK or an error code (message set).
int check_pool(const kunserve_kv_pool* pool, bool need_vec_align);

// ------------------------------------------------------ device helpers

__device__ __forceinline__ float bits_to_f32(int x) {
  return __builtin_bit_cast(float, x);
}
__device__ __forceinline__ int f32_to_bits(float x) {
  return __builtin_bit_cast(int, x);
}

// DPP lane moves within a row of 16 lanes. The row-local butterfly below
// uses quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1] (xor 2),
// row_half_mirror (pairs lane i with 7-i of each 8) and row_mirror (pairs
// lane i with 15-i of the row). After the four steps every lane of a
// 16-lane row holds the row total.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return bits_to_f32(
      __builtin_amdgcn_mov_dpp(f32_to_bits(x), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  return x;
}

__device__ __forceinline__ float row8_sum(float x) {
  x += dpp_f32<0xB1>(x);
  x += dpp_f32<0x4E>(x);
  x += dpp_f32<0x141>(x);
  return x;
}

// Sum over groups of LANES consecutive lanes (LANES in {8, 16, 32, 64}).
template <int LANES>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (LANES == 8) {
    return row8_sum(x);
  } else if constexpr (LANES == 16) {
    return row16_sum(x);
  } else if constexpr (LANES == 32) {
    x = row16_sum(x);
    return x + __shfl_xor(x, 16);
  } else {
    x = row16_sum(x);
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
  }
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// 16-byte global load / store of fp16x8.
__device__ __forceinline__ f16x8 load_f16x8(const f16* p) {
  return *reinterpret_cast<const f16x8*>(p);
}
// Non-temporal 16-byte load for data that is streamed once.
__device__ __forceinline__ f16x8 load_f16x8_nt(const f16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p));
}
__device__ __forceinline__ void store_f16x8(f16* p, f16x8 v) {
  *reinterpret_cast<f16x8*>(p) = v;
}

// Dot product of 8 fp16 pairs accumulated in fp32 (v_dot2_f32_f16).
__device__ __forceinline__ float dot8(f16x8 a, f16x8 b, float acc) {
  const fp16x2* pa = reinterpret_cast<const fp16x2*>(&a);
  const fp16x2* pb = reinterpret_cast<const fp16x2*>(&b);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(pa[i], pb[i], acc, false);
  return acc;
}
// The same for bf16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b, float acc) {
  const bf16x2* pa = reinterpret_cast<const bf16x2*>(&a);
  const bf16x2* pb = reinterpret_cast<const bf16x2*>(&b);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2_f32_bf16(pa[i], pb[i], acc, false);
  return acc;
}

// ------------------------------------------------ element-type generics
// The attention kernels are templates over the 16-bit element type T (f16
// or bf16). Pools, q and outputs are addressed as 16-bit storage; these
// helpers give the typed vector view and the matching MFMA.
template <typename T> struct Vec;
template <> struct Vec<f16> { typedef f16x8 v8; typedef f16x4 v4; };
template <> struct Vec<bf16> { typedef bf16x8 v8; typedef bf16x4 v4; };

template <typename T>
__device__ __forceinline__ typename Vec<T>::v8 load_v8(const void* p) {
  return *reinterpret_cast<const typename Vec<T>::v8*>(p);
}
template <typename T>
__device__ __forceinline__ typename Vec<T>::v8 load_v8_nt(const void* p) {
  return __builtin_bit_cast(typename Vec<T>::v8,
                            __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace kunserve
