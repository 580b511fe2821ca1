// Dense D x D rotation y = x @ R (or x @ R^T) for gfx950.
//
// Replaces the fp32 matmuls of oscar_ascend/backend.py:371 (q @ R_k) and :382
// (out_rot @ R_v^T).  One wave computes a 32 x 32 output tile with
// v_mfma_f32_32x32x16_bf16 over a three-term split of both operands
// (x_hi R_hi + x_lo R_hi + x_hi R_lo, hi = bf16(v), lo = bf16(v - hi)), which keeps
// the product error below 2^-16 of |x||R| with fp32 accumulation; the result is
// rounded once to the output dtype.
#include "common.h"

namespace oscar {

namespace {

struct Split { __bf16 hi, lo; };

__device__ __forceinline__ Split split_bf16(float v) {
  unsigned short h = f32_to_bf16_bits(v);
  float hv = bf16_bits_to_f32(h);
  unsigned short l = f32_to_bf16_bits(v - hv);
  return {__builtin_bit_cast(__bf16, h), __builtin_bit_cast(__bf16, l)};
}

__global__ __launch_bounds__(64) void rotate_kernel(oscar_rotate_args_v1 a) {
  const int lane = threadIdx.x, m = lane & 31, g = lane >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  const int col0 = blockIdx.y * 32;
  const int64_t D = a.head_dim;
  const int64_t row = row0 + m;
  const bool row_ok = row < a.rows;
  f32x16 acc = {};
  for (int k0 = 0; k0 < D; k0 += 16) {
    bf16x8 xh, xl, rh, rl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = k0 + 8 * g + e;
      float xv = row_ok ? load_elem(a.x, a.x_dtype, row * a.x_stride_row + k) : 0.f;
      const Split xs = split_bf16(xv);
      xh[e] = xs.hi;
      xl[e] = xs.lo;
      // B[k][n] = R[k][col] or R^T[k][col] = R[col][k]
      const int col = col0 + m;
      float rv = a.transpose ? a.r[(int64_t)col * D + k] : a.r[(int64_t)k * D + col];
      const Split rs = split_bf16(rv);
      rh[e] = rs.hi;
      rl[e] = rs.lo;
    }
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, rh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl, rh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, rl, acc, 0, 0, 0);
  }
  // D[i][j]: lane = j + 32*((i/4)%2), register = (i%4) + 4*(i/8); here i = row, j = col
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r >> 2) + 4 * g + (r & 3);
    const int64_t orow = row0 + i;
    if (orow < a.rows) store_elem(a.out, a.out_dtype, orow * a.out_stride_row + col0 + m, acc[r]);
  }
}

}  // namespace

}  // namespace oscar

using namespace oscar;

extern "C" int oscar_rotate_v1(const oscar_rotate_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_rotate_v1: null args");
  const oscar_rotate_args_v1& a = *args;
  if (a.rows == 0) return 0;
  if (a.rows < 0 || !a.x || !a.r || !a.out) return fail(-22, "oscar_rotate_v1: invalid arguments");
  if (a.head_dim % 32 || a.head_dim <= 0 || a.head_dim > 1024)
    return fail(-22, "oscar_rotate_v1: head_dim must be a multiple of 32");
  if (a.x_stride_row < a.head_dim || a.out_stride_row < a.head_dim)
    return fail(-22, "oscar_rotate_v1: row strides smaller than head_dim");
  if (a.rows > (int64_t)1 << 36) return fail(-22, "oscar_rotate_v1: too many rows");
  dim3 grid((unsigned)((a.rows + 31) / 32), (unsigned)(a.head_dim / 32));
  hipLaunchKernelGGL(rotate_kernel, grid, dim3(64), 0, (hipStream_t)stream, a);
  OSCAR_CHECK_LAUNCH("rotate_kernel");
  return 0;
}
