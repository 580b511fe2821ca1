// Dense D x D rotation y = x @ R (or x @ R^T) for gfx950.
//
// Replaces the fp32 matmuls of oscar_ascend/backend.py:371 (q @ R_k) and :382
// (out_rot @ R_v^T).  A workgroup of four waves computes a 32 x 32 output tile with
// v_mfma_f32_32x32x16_bf16 over a three-term split of both operands
// (x_hi R_hi + x_lo R_hi + x_hi R_lo, hi = bf16(v), lo = bf16(v - hi)), which keeps
// the product error below 2^-16 of |x||R| with fp32 accumulation; each wave takes
// a quarter of the contraction, the four partial tiles are summed in LDS and the
// result is rounded once to the output dtype.
//
// The input dtype, the output dtype and the transpose flag are template
// parameters, so the operand loads of all K-steps are plain vector loads with no
// branch between them, issued together ahead of the MFMAs.
#include "common.h"

namespace oscar {

namespace {

typedef __bf16 __attribute__((ext_vector_type(2))) bf16x2;
typedef float __attribute__((ext_vector_type(2))) f32x2;

// hi/lo bf16 split of 8 floats into two MFMA operands
__device__ __forceinline__ void split8(const float* v, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2 a = {v[2 * i], v[2 * i + 1]};
    const bf16x2 hb = __builtin_convertvector(a, bf16x2);
    const f32x2 hv = __builtin_convertvector(hb, f32x2);
    h[i] = __builtin_bit_cast(unsigned, hb);
    l[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(a - hv, bf16x2));
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

template <int D, int XT, int OT, bool TR>
__global__ __launch_bounds__(256) void rotate_kernel(oscar_rotate_args_v1 a) {
  constexpr int KS = D / 16 / 4;  // K-steps per wave
  const int lane = threadIdx.x & 63, m = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  const int col0 = blockIdx.y * 32;
  const int64_t row = row0 + m;
  const bool row_ok = row < a.rows;
  const int64_t xrow = (row_ok ? row : row0) * a.x_stride_row;  // row0 < rows always
  const int col = col0 + m;
  // all operand loads of this wave's K range first
  float xv[KS][8], rv[KS][8];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int kk = (wave * KS + s) * 16 + 8 * g;
    load8<XT>(a.x, xrow + kk, xv[s]);
    // B[k][n]: R[k][col], or R^T[k][col] = R[col][k] (contiguous in k)
    if constexpr (TR) {
      load8<OSCAR_F32>(a.r, (int64_t)col * D + kk, rv[s]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) rv[s][e] = a.r[(int64_t)(kk + e) * D + col];
    }
  }
  f32x16 acc = {};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (!row_ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[s][e] = 0.f;
    }
    bf16x8 xh, xl, rh, rl;
    split8(xv[s], xh, xl);
    split8(rv[s], rh, rl);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, rh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl, rh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, rl, acc, 0, 0, 0);
  }
  // sum of the four wave tiles (register order), then the store
  __shared__ f32x4 part[3][4][64];
  if (wave > 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      part[wave - 1][q][lane] = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 v = part[w][q][lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[4 * q + j] += v[j];
    }
  // D[i][j]: lane = j + 32*((i/4)%2), register = (i%4) + 4*(i/8); here i = row, j = col
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r >> 2) + 4 * g + (r & 3);
    const int64_t orow = row0 + i;
    if (orow < a.rows) store_elem(a.out, OT, orow * a.out_stride_row + col, acc[r]);
  }
}

template <int D, int XT, int OT>
void launch_tr(const oscar_rotate_args_v1& a, dim3 grid, hipStream_t s) {
  if (a.transpose) hipLaunchKernelGGL((rotate_kernel<D, XT, OT, true>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((rotate_kernel<D, XT, OT, false>), grid, dim3(256), 0, s, a);
}

template <int D, int XT>
void launch_out(const oscar_rotate_args_v1& a, dim3 grid, hipStream_t s) {
  if (a.out_dtype == OSCAR_BF16) launch_tr<D, XT, OSCAR_BF16>(a, grid, s);
  else if (a.out_dtype == OSCAR_F16) launch_tr<D, XT, OSCAR_F16>(a, grid, s);
  else launch_tr<D, XT, OSCAR_F32>(a, grid, s);
}

template <int D>
void launch_in(const oscar_rotate_args_v1& a, dim3 grid, hipStream_t s) {
  if (a.x_dtype == OSCAR_BF16) launch_out<D, OSCAR_BF16>(a, grid, s);
  else if (a.x_dtype == OSCAR_F16) launch_out<D, OSCAR_F16>(a, grid, s);
  else launch_out<D, OSCAR_F32>(a, grid, s);
}

}  // namespace

}  // namespace oscar

using namespace oscar;

extern "C" int oscar_rotate_v1(const oscar_rotate_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_rotate_v1: null args");
  const oscar_rotate_args_v1& a = *args;
  if (a.rows == 0) return 0;
  if (a.rows < 0 || !a.x || !a.r || !a.out) return fail(-22, "oscar_rotate_v1: invalid arguments");
  if (a.head_dim != 128 && a.head_dim != 256)
    return fail(-22, "oscar_rotate_v1: head_dim %lld unsupported (128/256)", (long long)a.head_dim);
  if (a.x_stride_row < a.head_dim || a.out_stride_row < a.head_dim)
    return fail(-22, "oscar_rotate_v1: row strides smaller than head_dim");
  if ((a.x_dtype != OSCAR_F32 && a.x_dtype != OSCAR_F16 && a.x_dtype != OSCAR_BF16) ||
      (a.out_dtype != OSCAR_F32 && a.out_dtype != OSCAR_F16 && a.out_dtype != OSCAR_BF16))
    return fail(-22, "oscar_rotate_v1: unsupported dtype");
  // rows are read as 16-byte vectors (8 elements of bf16/fp16, 2 x 4 of fp32)
  const int esz = a.x_dtype == OSCAR_F32 ? 4 : 2;
  if ((((uintptr_t)a.x) & 15) || ((a.x_stride_row * esz) & 15) || (((uintptr_t)a.r) & 15))
    return fail(-22, "oscar_rotate_v1: x rows and R must be 16-byte aligned");
  if (a.rows > (int64_t)1 << 36) return fail(-22, "oscar_rotate_v1: too many rows");
  dim3 grid((unsigned)((a.rows + 31) / 32), (unsigned)(a.head_dim / 32));
  hipStream_t s = (hipStream_t)stream;
  if (a.head_dim == 256) launch_in<256>(a, grid, s);
  else launch_in<128>(a, grid, s);
  OSCAR_CHECK_LAUNCH("rotate_kernel");
  return 0;
}
