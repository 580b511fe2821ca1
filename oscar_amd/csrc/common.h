// Shared device/host helpers for the gfx950 OSCAR kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/oscar_amd.h"

namespace oscar {

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;
typedef __attribute__((ext_vector_type(2))) int i32x2;

// ---------------------------------------------------------------- host errors
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define OSCAR_CHECK_LAUNCH(name)                                                   \
  do {                                                                             \
    hipError_t e_ = hipGetLastError();                                             \
    if (e_ != hipSuccess) return ::oscar::fail(-5, "%s launch: %s", name,         \
                                               hipGetErrorString(e_));            \
  } while (0)

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_bits_to_f32(unsigned short b) {
  return __uint_as_float(((unsigned)b) << 16);
}
__device__ __forceinline__ unsigned short f32_to_bf16_bits(float x) {
  // round to nearest even; NaN stays NaN (quiet)
  unsigned u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}
__device__ __forceinline__ unsigned short f32_to_f16_bits(float x) {
  return __half_as_ushort(__float2half_rn(x));
}
__device__ __forceinline__ float f16_bits_to_f32(unsigned short b) {
  return __half2float(__ushort_as_half(b));
}

// load element i of a dense row in dtype (F32/F16/BF16) as float
__device__ __forceinline__ float load_elem(const void* base, int32_t dtype, int64_t i) {
  if (dtype == OSCAR_BF16) return bf16_bits_to_f32(((const unsigned short*)base)[i]);
  if (dtype == OSCAR_F16) return f16_bits_to_f32(((const unsigned short*)base)[i]);
  return ((const float*)base)[i];
}
__device__ __forceinline__ void store_elem(void* base, int32_t dtype, int64_t i, float x) {
  if (dtype == OSCAR_BF16) ((unsigned short*)base)[i] = f32_to_bf16_bits(x);
  else if (dtype == OSCAR_F16) ((unsigned short*)base)[i] = f32_to_f16_bits(x);
  else ((float*)base)[i] = x;
}

// 8 consecutive elements (16-byte aligned for 2-byte types, 2 x 16 bytes for fp32)
// of dtype DT as floats
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t i, float* v) {
  if constexpr (DT == OSCAR_F32) {
    const f32x4 a = *(const f32x4*)((const float*)base + i);
    const f32x4 b = *(const f32x4*)((const float*)base + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[4 + e] = b[e]; }
  } else {
    const u32x4 a = *(const u32x4*)((const uint16_t*)base + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned w = a[e];
      if constexpr (DT == OSCAR_BF16) {
        v[2 * e] = __uint_as_float(w << 16);
        v[2 * e + 1] = __uint_as_float(w & 0xffff0000u);
      } else {
        v[2 * e] = f16_bits_to_f32(w & 0xffff);
        v[2 * e + 1] = f16_bits_to_f32(w >> 16);
      }
    }
  }
}

// ---------------------------------------------------------------- wave helpers
// x of another lane of the same 16-lane row, by a DPP control (quad_perm, mirrors)
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within 16

// x of lane l ^ 32 (v_permlane32_swap: each half receives the other half's values)
__device__ __forceinline__ float swap_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  // r[0]: lanes 0-31 keep their value, lanes 32-63 receive lanes 0-31's;
  // r[1]: lanes 0-31 receive lanes 32-63's, lanes 32-63 keep theirs.
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// x of lane l ^ 16 (ds_swizzle bit mode: and mask 0x1f, xor mask 0x10; the pattern is
// an immediate, so no lane-address register stays live across loops)
__device__ __forceinline__ float swizzle_xor16(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}

// all-lane reduction of a full wave under a commutative, associative op: xor 1, xor 2
// within each quad, the half mirror (quad pairs) and the mirror (8-lane halves) within
// each 16-lane row, then lane l ^ 16 and l ^ 32
template <class Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
  x = op(x, dpp_row<kDppXor1>(x));
  x = op(x, dpp_row<kDppXor2>(x));
  x = op(x, dpp_row<kDppHalfMirror>(x));
  x = op(x, dpp_row<kDppMirror>(x));
  x = op(x, swizzle_xor16(x));
  return op(x, swap_halves(x));
}

// all-lane max / min of a full wave (exact, so the order is free)
template <bool MAX>
__device__ __forceinline__ float wave_extreme(float x) {
  return wave_reduce(x, [](float a, float b) { return MAX ? fmaxf(a, b) : fminf(a, b); });
}
__device__ __forceinline__ float wave_max(float x) { return wave_extreme<true>(x); }
__device__ __forceinline__ float wave_min(float x) { return wave_extreme<false>(x); }

// s_waitcnt lgkmcnt(0) leaving vmcnt/expcnt at their maxima (gfx9 encoding):
// waits for this wave's LDS traffic without draining outstanding global loads.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

}  // namespace oscar
