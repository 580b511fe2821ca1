// INT2 write path for gfx950: rotate, sort-clip, quantize, pack, scatter, staging.
//
// Replaces oscar_ascend/kernels/store_kernel.py:54-102 / :166-279 and the
// host-side pieces of oscar_ascend/backend.py around them (_rotate_clip
// :130-148, do_kv_cache_update :151-198, _staging_write :513-555, and the
// read-path rotations :370-373).
//
// The stored bytes are those of the correctly rounded rotation y = x @ R (fp32 result
// of the exact sum), clipped and quantized as the reference does.  Two paths:
//
//   calls of <= kFusedTokens tokens (decode / MTP steps): store_small_kernel, one
//   launch of (32-column slice, group of 8 vectors) workgroups; y in fp64 (exact
//   products, one rounding), winners by scanning the call's slot_mapping.  Under
//   oscar_decode_write_v1 the launch stops after the rotation (deferred: pending owner
//   tags on the seats it rewrites) and the decode's merge launch quantizes
//   (store_quant.h).
//
//   larger calls: store_prep_kernel (last-writer claims, window flags, fp16 planes of R),
//   store_fused_kernel (MFMA rotation into LDS, then per vector: read-path copy,
//   certification that every quantizer decision taken on the MFMA result is the one
//   the exact y takes, quantization; the FP32 window copies of its vectors are y~ itself,
//   within the rotation bound e of y), store_exact_kernel (fp64 y for the vectors that
//   were not certified).
//
// Claim epochs live on the device in two int64 words so that a captured graph
// replays with fresh epochs and no extra launch: the prep kernel uses
// E = word0 + 1 and stores E in word1; the fused kernel reads word1 and copies it
// to word0 for the next call.
#include <atomic>
#include <type_traits>

#include "common.h"
#include "store_quant.h"

namespace oscar {

namespace {

// Calls of at most kFusedTokens tokens (decode and MTP steps): one launch of
// workgroups (slice, vector group).  The vectors of a kind -- K and V rows (token, kv
// head), query rows (token, q head) -- are cut into groups of kSmallVecs consecutive
// rows; a workgroup rotates one group for one slice of kSmallCols output columns, so
// that it streams D x kSmallCols of R (32 KB) for kSmallVecs vectors.  Thread
// (column pair cp, part kp) holds rows kp + kSmallParts * i of the slice's two
// columns in registers, the products accumulate in fp64 (exact: bf16/fp16/fp32
// inputs times fp32) and the kSmallParts parts of each output are added in order in
// LDS, so the fp32 result is the correctly rounded one.  Query slices go to
// query_rot.  K / V slices go to the read-path copies and to the workspace; the last
// slice workgroup of a group to arrive (one counter per group that atomicInc wraps
// back to zero) reads the group's vectors back and quantizes, packs and scatters
// them in place, one wave per vector (quant_vector; destinations and winners by
// scanning the call's slot_mapping, computed by every slice workgroup while its
// slice stores complete).  The slices pass through the workspace with agent-scope
// stores and loads, which bypass the per-XCD L2, ordered by the store wait, the
// barrier and the counter; an agent-scope fence would instead write back and
// invalidate the whole L2 in every workgroup.
constexpr int64_t kFusedTokens = 64;
constexpr int kSmallVecs = 8;     // vectors per workgroup (one quantizing wave each)
constexpr int kSmallCols = 32;    // output columns per workgroup
constexpr int kSmallParts = 32;   // parts of the contraction (16 column pairs x 32 = 512 threads)
constexpr int kSmallThreads = 512;
static_assert(kFusedTokens <= 64, "dest_loads reads one slot of the call per lane");

// vector groups of each kind of a small call
__host__ __device__ inline int64_t small_groups(int64_t vectors) { return (vectors + kSmallVecs - 1) / kSmallVecs; }

template <int D, int XT>
__global__ __launch_bounds__(kSmallThreads) void store_small_kernel(StoreParams p) {
  constexpr int NS = D / kSmallCols;   // slices of a vector
  constexpr int RPT = D / kSmallParts;  // rows of R per thread (consecutive)
  static_assert(kSmallVecs * kSmallCols <= kSmallThreads && kSmallThreads == 16 * kSmallParts && RPT % 2 == 0,
                "slice shape");
  const oscar_store_args_v1& a = p.a;
  const int64_t hk = a.cache.num_kv_heads;
  const int64_t nkv = a.num_tokens * hk, nq = a.num_tokens * a.num_q_heads;
  const int64_t gkv = small_groups(nkv);
  const int c0 = blockIdx.x * kSmallCols;
  const int64_t gy = blockIdx.y;
  const int kind = gy < gkv ? KIND_K : (gy < 2 * gkv ? KIND_V : KIND_Q);
  const int64_t grp = kind == KIND_K ? gy : (kind == KIND_V ? gy - gkv : gy - 2 * gkv);
  const FastDiv& dh = kind == KIND_Q ? p.div_hq : p.div_hk;  // vector -> token, head
  const int64_t count = kind == KIND_Q ? nq : nkv;
  const int64_t v0 = grp * kSmallVecs;  // first vector (token * heads + head) of the group
  const int nv = count - v0 < kSmallVecs ? (int)(count - v0) : kSmallVecs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cp = tid & 15, kp = tid >> 4;
  const bool kv = kind != KIND_Q;
  const void* src = kind == KIND_K ? a.key : (kind == KIND_V ? a.value : a.query);
  const int64_t src_stride = kind == KIND_K ? a.key_stride_token
                           : (kind == KIND_V ? a.value_stride_token : a.query_stride_token);
  const float* R = (kind == KIND_V) ? a.rv : a.rk;
  void* rot_out = kind == KIND_K ? a.key_rot : (kind == KIND_V ? a.value_rot : a.query_rot);

  __shared__ __attribute__((aligned(16))) double s_x[kSmallVecs][D];
  __shared__ double s_red[kSmallParts][kSmallVecs * kSmallCols];
  __shared__ int s_last;
  // this thread's rows kp * RPT + i of the slice's columns c0 + 2 cp, + 1: issued
  // first, used after the barrier
  f32x2 r2[RPT];
  if (R != nullptr) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) r2[i] = *(const f32x2*)(R + (int64_t)(kp * RPT + i) * D + c0 + 2 * cp);
  }
  // the group's input vectors (fp64 in LDS; rows past nv are zero)
  for (int e = tid; e < kSmallVecs * (D / 8); e += kSmallThreads) {
    const int v = e / (D / 8), k8 = (e % (D / 8)) * 8;
    float xv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (v < nv) {
      const uint32_t vi = (uint32_t)(v0 + v), t = fdiv(vi, dh);
      load8<XT>(src, (int64_t)t * src_stride + (int64_t)(vi - t * dh.d) * D + k8, xv);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s_x[v][k8 + j] = (double)xv[j];
  }
  // the destination loads of this wave's K / V vector (the token of vector v0 +
  // wave): out with the operands, used after the products
  const uint32_t vw = (uint32_t)(v0 + wave);
  const int64_t t = fdiv(vw, p.div_hk), h = vw - (uint32_t)t * p.div_hk.d;
  DestLoads dl{};
  if (kv && !p.deferred && wave < nv) dl = dest_loads(p, t);
  __syncthreads();
  double acc[kSmallVecs][2];
  if (R != nullptr) {
#pragma unroll
    for (int v = 0; v < kSmallVecs; ++v) acc[v][0] = acc[v][1] = 0.0;
#pragma unroll
    for (int i = 0; i < RPT; i += 2) {
      const double r00 = r2[i][0], r01 = r2[i][1], r10 = r2[i + 1][0], r11 = r2[i + 1][1];
#pragma unroll
      for (int v = 0; v < kSmallVecs; ++v) {
        const double2 x = *(const double2*)&s_x[v][kp * RPT + i];
        acc[v][0] = fma(x.y, r10, fma(x.x, r00, acc[v][0]));
        acc[v][1] = fma(x.y, r11, fma(x.x, r01, acc[v][1]));
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < kSmallVecs; ++v)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[v][j] = kp == 0 ? s_x[v][c0 + 2 * cp + j] : 0.0;
  }
  // the parts to LDS; thread e < kSmallVecs * kSmallCols adds the parts of output e
  // (vector e / kSmallCols, column e % kSmallCols) in order
#pragma unroll
  for (int v = 0; v < kSmallVecs; ++v)
#pragma unroll
    for (int j = 0; j < 2; ++j) s_red[kp][v * kSmallCols + 2 * cp + j] = acc[v][j];
  __syncthreads();
  if (tid < kSmallVecs * kSmallCols) {
    double sum = 0.0;
#pragma unroll 8
    for (int w = 0; w < kSmallParts; ++w) sum += s_red[w][tid];
    const int v = tid / kSmallCols, col = c0 + tid % kSmallCols;
    if (v < nv) {
      const float y = (float)sum;
      const int64_t vi = v0 + v;
      if (rot_out != nullptr) store_elem(rot_out, XT, vi * D + col, y);
      // agent-coherent stores (past this XCD's L2), read back the same way below
      if (kv) __hip_atomic_store(p.y + ((int64_t)kind * nkv + vi) * D + col, y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!kv) return;
  if (p.deferred) {
    // the seats of the call's valid tokens get the pending tag; the quantization
    // writes their final tags (every such seat has a last writer among the tokens)
    if (kind == KIND_K && blockIdx.x == 0 && tid < nv && a.stage_mode != OSCAR_STAGE_NONE) {
      const int64_t slot = a.slot_mapping[fdiv((uint32_t)(v0 + tid), p.div_hk)];
      if (slot >= 0 && slot < p.capacity) a.staging.owner[seat_of(p, slot)] = kPendingTag;
    }
    return;
  }
  Dest dest{};
  if (wave < nv) dest = dest_finish(p, kind, t, dl);
  // the slice is written (stores complete before the barrier): count it in; the last
  // of the group's slices to arrive goes on
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if constexpr (NS > 1) {
    if (tid == 0) s_last = atomicInc(&a.arrivals[(int64_t)kind * gkv + grp], NS - 1) == NS - 1;
    __syncthreads();
    if (!s_last) return;
  }
  if (wave >= nv) return;
  const float* yv = p.y + ((int64_t)kind * nkv + vw) * D + 4 * (lane < D / 4 ? lane : 0);
  f32x4 x4;
#pragma unroll
  for (int j = 0; j < 4; ++j) x4[j] = __hip_atomic_load(yv + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  quant_vector<D>(p, kind, t, h, dest, x4);
}


// Certified fp16 scale bits of the quantizer for (vmax, vmin): RN(vmax - vmin) / 3 (RN),
// floored at 2^-14, to fp16 (RN) -- each step monotone in vmax - vmin.
__device__ __forceinline__ unsigned short scale_bits_of(float vmax, float vmin) {
  float scale = __fdiv_rn(vmax - vmin, 3.0f);
  if (!(scale > 0x1p-14f)) scale = 0x1p-14f;
  return f32_to_f16_bits(scale);
}
__device__ __forceinline__ int code_of(float x, float z16, float s16) {
  const float q = fminf(fmaxf(floorf(__fdiv_rn(x - z16, s16) + 0.5f), 0.f), 3.f);
  return (int)q;
}

// ---- 16-lane rows: a wave quantizes four vectors at once, lane l of a row holding
// elements [l E, (l + 1) E) of its vector (E = D / 16)
template <int CTRL>
__device__ __forceinline__ int dpp_row_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, true);
}
// NaN-propagating minimum / maximum over the 16-lane row
__device__ __forceinline__ float row_minimum(float x) {
  x = __builtin_elementwise_minimum(x, dpp_row<kDppXor1>(x));
  x = __builtin_elementwise_minimum(x, dpp_row<kDppXor2>(x));
  x = __builtin_elementwise_minimum(x, dpp_row<kDppHalfMirror>(x));
  return __builtin_elementwise_minimum(x, dpp_row<kDppMirror>(x));
}
__device__ __forceinline__ float row_maximum(float x) {
  x = __builtin_elementwise_maximum(x, dpp_row<kDppXor1>(x));
  x = __builtin_elementwise_maximum(x, dpp_row<kDppXor2>(x));
  x = __builtin_elementwise_maximum(x, dpp_row<kDppHalfMirror>(x));
  return __builtin_elementwise_maximum(x, dpp_row<kDppMirror>(x));
}
__device__ __forceinline__ int row_sum(int x) {
  x += dpp_row_i<kDppXor1>(x);
  x += dpp_row_i<kDppXor2>(x);
  x += dpp_row_i<kDppHalfMirror>(x);
  return x + dpp_row_i<kDppMirror>(x);
}
// the predicate holds on every lane of this lane's row
__device__ __forceinline__ bool row_all(bool pred) {
  const uint64_t m = __ballot(pred);
  return ((m >> (threadIdx.x & 48)) & 0xffffull) == 0xffffull;
}

// the median of three (v_med3_u32)
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t row_min_u32(uint32_t x) {
  x = min(x, (uint32_t)dpp_row_i<kDppXor1>((int)x));
  x = min(x, (uint32_t)dpp_row_i<kDppXor2>((int)x));
  x = min(x, (uint32_t)dpp_row_i<kDppHalfMirror>((int)x));
  return min(x, (uint32_t)dpp_row_i<kDppMirror>((int)x));
}
__device__ __forceinline__ uint32_t row_max_u32(uint32_t x) {
  x = max(x, (uint32_t)dpp_row_i<kDppXor1>((int)x));
  x = max(x, (uint32_t)dpp_row_i<kDppXor2>((int)x));
  x = max(x, (uint32_t)dpp_row_i<kDppHalfMirror>((int)x));
  return max(x, (uint32_t)dpp_row_i<kDppMirror>((int)x));
}

// idx-th smallest |y| of the row's D values (the sort-clip threshold, backend.py:140-145),
// on the magnitude bits (their order is that of |y|; the row is finite): the answer a is
// the largest v with count(|y| < v) <= idx, i.e. the (D - idx)-th largest element.
// Bisection of [lo, hi) with a in [lo, hi): hi = row maximum + 1, lo = the row minimum of
// each lane's k-th largest, k = 1 while D - idx <= 16, 2 while <= 32 (each of the 16
// lanes holds k elements >= lo, so at least D - idx do and a >= lo), else 0.  c_lo .. c_hi
// bound the ranks inside the interval; a row whose interval holds exactly one element
// stops there and takes that element (the row's smallest element at or above lo), a row
// whose interval is one value wide takes lo (ties).  The loop runs while any row of the
// wave is open.
template <int E>
__device__ float row_kth_abs(const float* y, int idx) {
  constexpr int N = 16 * E;
  uint32_t u[E];
  uint32_t m1 = 0, m2 = 0;  // this lane's largest and second largest
#pragma unroll
  for (int j = 0; j < E; ++j) {
    u[j] = __float_as_uint(y[j]) & 0x7fffffffu;
    m2 = max(m2, min(m1, u[j]));
    m1 = max(m1, u[j]);
  }
  const int need = N - idx;
  uint32_t lo = row_min_u32(need <= 16 ? m1 : (need <= 32 ? m2 : 0u));
  uint32_t hi = row_max_u32(m1) + 1u;  // <= 2^31: every element and candidate is below
  int c_lo = 0, c_hi = N;  // c_lo: a lower bound of count(|y| < lo) until lo first moves
  bool open = hi - lo > 1;
  auto bisect = [&]() {
    // an open row has lo < mid < hi: med3(u, mid - 1, mid) is mid - 1 for u < mid and mid
    // otherwise, so the lane's sum is E (mid - 1) + count(u >= mid) (mod 2^32)
    const uint32_t mid = lo + ((hi - lo) >> 1);
    uint32_t s = 0;
#pragma unroll
    for (int j = 0; j < E; j += 2) s += med3_u32(u[j], mid - 1u, mid) + med3_u32(u[j + 1], mid - 1u, mid);
    const int cnt = row_sum(E - (int)(s - (uint32_t)E * (mid - 1u)));  // count(|y| < mid)
    const bool up = open && cnt <= idx, down = open && cnt > idx;
    lo = up ? mid : lo;
    c_lo = up ? cnt : c_lo;
    hi = down ? mid : hi;
    c_hi = down ? cnt : c_hi;
    open = hi - lo > 1 && c_hi - c_lo > 1;
  };
  // two steps per test of the wave (a closed row's step changes nothing)
  while (__any(open)) {
    bisect();
    bisect();
  }
  // the one element of [lo, hi) when c_hi - c_lo == 1 is the row's smallest element at or
  // above lo (u - lo wraps past 2^31 for the elements below lo)
  uint32_t dmin = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < E; ++j) dmin = min(dmin, u[j] - lo);
  dmin = row_min_u32(dmin);
  return __uint_as_float(c_hi - c_lo == 1 ? lo + dmin : lo);
}

// Certify and quantize the rows' vectors from y~ (lane: y[E] of its row's vector).  The
// bound on |y~_j - y_j| is taken row-uniform: eb = ex + 2^-22 max_j |y~_j| (ex: the row's
// rotation term plus 2^-126), at least every element's own bound.  Every decision the
// quantizer takes -- the sort-clip threshold (order statistics move by at most eb), the
// fp16 scale and zero (from the intervals of vmin and vmax) and each code -- is evaluated
// over the whole interval y~ +- eb; the quantizer's steps are monotone, so one outcome
// over the interval means y gives the same bytes.  Certified rows with write != 0 store
// their codes and meta (K slot kslot + 32 / V slot vslot); the function returns whether
// this lane's row was certified.
// CLIP false: the kind's sort clip is off (known at compile time, so that the common
// unclipped case carries no per-element clamps); true: tested at run time
template <int D, bool CLIP>
__device__ bool certify_quant16(const StoreParams& p, int kind, const float* y, float ex,
                                bool write, uint8_t* kslot, uint8_t* vslot) {
  constexpr int E = D / 16;
  const int l = threadIdx.x & 15;
  const float clip = kind == KIND_K ? p.a.k_clip_ratio : p.a.v_clip_ratio;
  const bool clipping = CLIP && clip > 0.f;
  // row extremes with NaN-propagating minimum / maximum: a NaN or inf anywhere makes eb
  // NaN or inf, and the row goes to the exact pass (which reproduces the reference)
  float vmin = y[0], vmax = y[0];
#pragma unroll
  for (int j = 1; j < E; ++j) {
    vmin = __builtin_elementwise_minimum(vmin, y[j]);
    vmax = __builtin_elementwise_maximum(vmax, y[j]);
  }
  vmin = row_minimum(vmin);
  vmax = row_maximum(vmax);
  const float eb = ex + __builtin_elementwise_maximum(fabsf(vmin), fabsf(vmax)) * 0x1p-22f;
  if (!row_all(eb <= 0x1.fffffep127f)) return false;
  float t_lo = INFINITY, t_hi = INFINITY;
  if (clipping) {
    int idx = (int)(clip * (float)D);
    if (idx > D - 1) idx = D - 1;
    const float t = row_kth_abs<E>(y, idx);
    const float et = eb + t * 0x1p-22f;
    t_lo = fmaxf(t - et, 0.f);
    t_hi = t + et;
  }
  // the ends of an element's interval, clipped like the values themselves: lower ends
  // into [-t_hi, t_lo], upper ends into [-t_lo, t_hi]; clipping and rounding are
  // monotone, so the row extremes of the ends are the ends of the row extremes
  auto lo_of = [&](float v) { return clipping ? fminf(fmaxf(v - eb, -t_hi), t_lo) : v - eb; };
  auto hi_of = [&](float v) { return clipping ? fminf(fmaxf(v + eb, -t_lo), t_hi) : v + eb; };
  const float vmin_lo = lo_of(vmin), vmin_hi = hi_of(vmin), vmax_lo = lo_of(vmax), vmax_hi = hi_of(vmax);
  const unsigned short s_a = scale_bits_of(vmax_lo, vmin_hi), s_b = scale_bits_of(vmax_hi, vmin_lo);
  const unsigned short z_a = f32_to_f16_bits(vmin_lo), z_b = f32_to_f16_bits(vmin_hi);
  // a zero of either sign is left to the exact pass: its sign bit follows y exactly
  if (s_a != s_b || z_a != z_b || (z_a & 0x7fff) == 0) return false;  // row-uniform
  const float s16 = f16_bits_to_f32(s_a), z16 = f16_bits_to_f32(z_a);
  const float inv = __builtin_amdgcn_rcpf(s16);
  // every element's q = (x - z) / s lies within the row's [q(vmin_lo), q(vmax_hi)]
  const float qm = fmaxf(fmaxf(fabsf((vmin_lo - z16) * inv), fabsf((vmax_hi - z16) * inv)), 1.f);
  if (!(qm <= 0x1p20f)) return false;  // also inf / NaN zero or scale (row-uniform)
  // Codes.  An element's (clipped) value lies within ew of its center yc (clipping is
  // 1-Lipschitz in the value and in the threshold, whose center is tc).  The quantizer's
  // RN(RN(x - z) / s) + 0.5 for any x there is within w = ew (1 / s) + 2^-19 max(|q|, 1)
  // of t = fma(yc - z, 1 / s, 0.5) (a few ulp of rounding, and 1 / s within one ulp), so
  // where t is farther than w from every integer, all of them share floor(t)'s code.
  const float tc = clipping ? 0.5f * (t_lo + t_hi) : INFINITY;
  const float ew = clipping ? eb + (0.5f * (t_hi - t_lo) + tc * 0x1p-22f) * (1.f + 0x1p-20f) : eb;
  const float w = ew * inv * (1.f + 0x1p-20f) + 0x1p-19f * qm;
  auto center = [&](int j) { return fmaf((clipping ? fminf(fmaxf(y[j], -tc), tc) : y[j]) - z16, inv, 0.5f); };
  auto code_at = [&](float t) {  // floor(t) clamped to [0, 3] (t truncated: equal after clamping)
    const int c = (int)t;
    return c < 0 ? 0 : (c > 3 ? 3 : c);
  };
  uint32_t packed = 0;  // byte b holds elements 4b..4b+3, two bits each (format.py:84-87)
  float nearest = INFINITY;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float t = center(j);
    nearest = __builtin_elementwise_minimum(nearest, fabsf(t - rintf(t)));
    packed |= (uint32_t)code_at(t) << (2 * j);
  }
  bool same = true;
  if (!(nearest > w)) {  // an element near a code boundary: the exact codes at both ends
    packed = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const float t = center(j);
      int code = code_at(t);
      if (!(fabsf(t - rintf(t)) > w)) {
        code = code_of(lo_of(y[j]), z16, s16);
        same &= code == code_of(hi_of(y[j]), z16, s16);
      }
      packed |= (uint32_t)code << (2 * j);
    }
  }
  if (!row_all(same)) return false;
  if (write) {
    uint8_t* dst = (kind == KIND_K ? kslot + 32 : vslot) + l * (E / 4);
    if constexpr (E == 16) *(uint32_t*)dst = packed;
    else if constexpr (E == 8) *(uint16_t*)dst = (uint16_t)packed;
    else *dst = (uint8_t)packed;
    if (l == 0) *(unsigned*)(kslot + (kind == KIND_K ? 0 : 4)) = (unsigned)s_a | ((unsigned)z_a << 16);
  }
  return true;
}

// ------------------------------------------------------------------ large calls
// Calls of more than kFusedTokens tokens, in three launches:
//
//   store_prep_kernel    one thread per token: the last-writer claims of its slot and
//                        seat (64-bit atomicMax of epoch<<24 | token), or the owner-tag
//                        invalidation of a standalone update, and the token's window flag
//                        (its position inside the sink / recent window of its request);
//                        and one block per 32-column block of R_k and R_v: its two fp16
//                        planes, scaled by a power of two per column, in MFMA B order.
//   store_fused_kernel   8 waves over runs of row blocks (32 vectors each) of one kind.
//                        Each wave keeps one 32-column block of R's planes in registers; a
//                        row block's x is
//                        staged in LDS as fp16 scaled by a power of two per vector (fp32
//                        inputs in two planes); v_mfma_f32_32x32x16_f16 forms y~ = x R in
//                        chains of kChainSteps K-steps whose sum is rounded once, into an LDS
//                        tile of whole vectors.  Then each wave takes vectors from the tile:
//                        read-path copy, destination, certification, quantization.
//   store_exact_kernel   the vectors that were not certified: y in fp64 (exact products,
//                        one final rounding), then the same quantizer (and their FP32
//                        window copies from that y).
//
// Error of y~ against y: the instruction's products are exact and it rounds C + (the
// sum of its 16 products) once to fp32 (measured on gfx950), so a chain of kChainSteps
// K-steps errs by <= kChainSteps * 2^-24 * sum_k |x_k R_kd|; the residual of R's two
// fp16 planes is <= 2^-22 |R_kd| per entry, that of fp32 x's two planes <= 2^-22 |x_k|,
// and the chain sum (exact two-sums, then one rounding) to fp32 (<= 2^-24 |y~|).  By Cauchy-Schwarz
// sum_k |x_k R_kd| <= ||x|| ||R_:d||, so with kChainSteps = 4
//     e = coef ||x|| ||R_:d|| + 2^-22 |y~|,  coef = 2^-20 (bf16 / fp16 x), 2^-19 (fp32 x)
// bounds |y~ - y| with a margin of 2 or more (and still holds if the instruction rounded
// twice).  Elements of x below 2^-31 max|x| or of R below 2^-31 max|R_:d| that fp16
// cannot hold exactly after scaling add < 2^-28 of the bound.
constexpr int kFusedThreads = 512;  // 8 waves
constexpr int kChainSteps = 4;      // K-steps per accumulation chain
constexpr int kExactThreads = 512;
constexpr int kExactGroup = 8;      // vectors per exact-pass group
constexpr int kReqLds = 2048;       // request tables of up to this many entries go to LDS

// power-of-two exponent s with m * 2^s in [2^14, 2^15) (m > 0 finite); 0 otherwise
__device__ __forceinline__ int fp16_exponent(float m) {
  if (!(m > 0.f) || !__builtin_isfinite(m)) return 0;
  int e;
  frexpf(m, &e);
  return 15 - e;
}

__device__ __forceinline__ unsigned f16_pair(float lo, float hi) {
  return (unsigned)f32_to_f16_bits(lo) | ((unsigned)f32_to_f16_bits(hi) << 16);
}

// fp16 planes of one 32-column block of R (which: 0 = R_k, 1 = R_v) in MFMA B order:
// fragment (s, lane n + 32 g) holds R[16 s + 8 g + j][32 cb + n] * 2^bexp, j < 8, as
// the rounded plane and the (exact) remainder rounded again.  The block's D x 32 entries
// are staged in LDS first (all loads in flight at once).
template <int D>
__device__ void rotation_planes(const StoreParams& p, int which, int cb) {
  constexpr int KS = D / 16;
  constexpr int NT = 256;                  // threads of the prep kernel
  constexpr int F4 = D * 8 / NT;           // float4 loads per thread
  const float* R = which ? p.a.rv : p.a.rk;
  const int tid = threadIdx.x, c = tid % 32, part = tid / 32;  // 8 parts of the rows
  __shared__ float s_r[D][33];
  __shared__ float s_mx[8][32], s_sq[8][32];
  __shared__ int s_e[32];
  f32x4 v[F4];
#pragma unroll
  for (int i = 0; i < F4; ++i) {  // float4 i of the thread: row (tid + i NT) / 8, columns 4 ((tid + i NT) % 8) ..
    const int q = tid + i * NT, k = q / 8, c0 = 32 * cb + 4 * (q % 8);
    if (R != nullptr) {
      v[i] = *(const f32x4*)(R + (int64_t)k * D + c0);
    } else {
      const int o = k - c0;  // identity: 1 where the column equals the row
      v[i] = f32x4{o == 0 ? 1.f : 0.f, o == 1 ? 1.f : 0.f, o == 2 ? 1.f : 0.f, o == 3 ? 1.f : 0.f};
    }
  }
#pragma unroll
  for (int i = 0; i < F4; ++i) {
    const int q = tid + i * NT, k = q / 8, cc = 4 * (q % 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) s_r[k][cc + j] = v[i][j];
  }
  __syncthreads();
  float mx = 0.f, sq = 0.f;
  for (int k = part; k < D; k += 8) {
    const float r = s_r[k][c];
    mx = fmaxf(mx, fabsf(r));
    sq = fmaf(r, r, sq);
  }
  s_mx[part][c] = mx;
  s_sq[part][c] = sq;
  __syncthreads();
  if (tid < 32) {
    for (int i = 1; i < 8; ++i) {
      mx = fmaxf(mx, s_mx[i][c]);
      sq += s_sq[i][c];
    }
    s_e[c] = fp16_exponent(mx);
    p.bexp[which * D + 32 * cb + c] = s_e[c];
    p.colnorm[which * D + 32 * cb + c] = sqrtf(sq);
  }
  __syncthreads();
  u32x4* out = p.planes + ((int64_t)(which * (D / 32) + cb) * KS) * 2 * 64;
  for (int f = tid; f < KS * 64; f += NT) {
    const int s = f / 64, lane = f % 64, n = lane % 32, g = lane / 32;
    const int e = s_e[n];
    u32x4 w0, w1;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int k = 16 * s + 8 * g + 2 * w;
      const float h0 = ldexpf(s_r[k][n], e), h1 = ldexpf(s_r[k + 1][n], e);
      const float q0 = f16_bits_to_f32(f32_to_f16_bits(h0)), q1 = f16_bits_to_f32(f32_to_f16_bits(h1));
      w0[w] = f16_pair(q0, q1);
      w1[w] = f16_pair(h0 - q0, h1 - q1);  // exact differences
    }
    out[(s * 2 + 0) * 64 + lane] = w0;
    out[(s * 2 + 1) * 64 + lane] = w1;
  }
}

// ---- claims, window flags and the rotation planes: blocks [0, 2 D / 32) take one
// column block of R_k or R_v, the blocks after them 256 tokens each
template <int D>
__global__ __launch_bounds__(256) void store_prep_kernel(StoreParams p) {
  const oscar_store_args_v1& a = p.a;
  constexpr int PB = 2 * (D / 32);  // plane blocks
  if (blockIdx.x < PB) {
    rotation_planes<D>(p, blockIdx.x / (D / 32), blockIdx.x % (D / 32));
    return;
  }
  const int64_t e0 = a.epoch_counter[0];
  const int64_t epoch = e0 < kMaxEpoch ? e0 + 1 : kMaxEpoch;
  if (blockIdx.x == PB && threadIdx.x == 0) a.epoch_counter[1] = epoch;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  const bool lds = window && a.num_reqs <= kReqLds;
  __shared__ int32_t s_qsl[kReqLds + 1];
  if (lds) {
    for (int r = threadIdx.x; r <= a.num_reqs; r += blockDim.x) s_qsl[r] = a.query_start_loc[r];
    __syncthreads();
  }
  const int64_t t = (int64_t)(blockIdx.x - PB) * blockDim.x + threadIdx.x;
  if (t >= a.num_tokens) return;
  const int64_t slot = a.slot_mapping[t];
  if (window) {
    // request of t: the last r < num_reqs with min(qsl[r], num_tokens) <= t (qsl is
    // non-decreasing); none -> length 0, end 0
    int lo = 0, hi = a.num_reqs;  // answer in [lo - 1, hi - 1]
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      int64_t st = lds ? s_qsl[mid] : a.query_start_loc[mid];
      if (st > a.num_tokens) st = a.num_tokens;
      if (st <= t) lo = mid + 1;
      else hi = mid;
    }
    const int r = lo - 1;
    const int64_t seq = r >= 0 ? a.seq_lens[r] : 0;
    const int64_t end = r >= 0 ? (lds ? s_qsl[r + 1] : a.query_start_loc[r + 1]) : 0;
    p.flags[t] = in_window(a, t, seq, end) ? 1 : 0;
  }
  if (slot < 0 || slot >= p.capacity) return;
  atomicMax((unsigned long long*)&a.slot_claims[slot], (unsigned long long)claim_value(epoch, t));
  if (a.stage_mode == OSCAR_STAGE_NONE) return;
  const int64_t seat = seat_of(p, slot);
  if (a.stage_mode == OSCAR_STAGE_INVALIDATE) a.staging.owner[seat] = -1;
  else atomicMax((unsigned long long*)&a.seat_claims[seat], (unsigned long long)claim_value(epoch, t));
}

// Destination of token t's vectors from the finished claims (slot already loaded)
__device__ __forceinline__ Dest claimed_dest(const StoreParams& p, int64_t t, int64_t slot, int32_t flag,
                                             int64_t epoch) {
  const oscar_store_args_v1& a = p.a;
  Dest d{};
  d.slot = slot;
  d.valid = slot >= 0 && slot < p.capacity;
  if (!d.valid) return d;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  const long long mine = claim_value(epoch, t);
  d.seat = a.stage_mode != OSCAR_STAGE_NONE ? seat_of(p, slot) : 0;
  d.slot_win = (long long)a.slot_claims[slot] == mine;
  d.seat_win = window && (long long)a.seat_claims[d.seat] == mine;
  d.keep = window && (flag & 1);
  return d;
}

// ---- x staging: a thread holds 16 consecutive elements of one vector
template <int XT>
struct XChunk {
  static constexpr int W = XT == OSCAR_F32 ? 4 : 2;  // 16-byte words
  u32x4 w[W];
  __device__ __forceinline__ void load(const void* base, int64_t i) {
    if constexpr (XT == OSCAR_F32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = *(const u32x4*)((const float*)base + i + 4 * k);
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k) w[k] = *(const u32x4*)((const uint16_t*)base + i + 8 * k);
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = u32x4{0u, 0u, 0u, 0u};
  }
  __device__ __forceinline__ void to_float(float* f) const {
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (XT == OSCAR_F32) {
          f[4 * k + e] = __uint_as_float(w[k][e]);
        } else if constexpr (XT == OSCAR_BF16) {
          f[8 * k + 2 * e] = __uint_as_float(w[k][e] << 16);
          f[8 * k + 2 * e + 1] = __uint_as_float(w[k][e] & 0xffff0000u);
        } else {
          f[8 * k + 2 * e] = f16_bits_to_f32((unsigned short)(w[k][e] & 0xffff));
          f[8 * k + 2 * e + 1] = f16_bits_to_f32((unsigned short)(w[k][e] >> 16));
        }
      }
  }
};

// max / sum over aligned groups of N consecutive lanes (N = 4, 8, 16); every lane of a
// group receives the same value (each step combines two equal-shaped halves, and + is
// commutative)
template <int N>
__device__ __forceinline__ float group_max(float x) {
  static_assert(N == 4 || N == 8 || N == 16, "group size");
  x = fmaxf(x, dpp_row<kDppXor1>(x));
  x = fmaxf(x, dpp_row<kDppXor2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp_row<kDppHalfMirror>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp_row<kDppMirror>(x));
  return x;
}
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 4 || N == 8 || N == 16, "group size");
  x += dpp_row<kDppXor1>(x);
  x += dpp_row<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp_row<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_row<kDppMirror>(x);
  return x;
}

template <int D, int XT>
__global__ __launch_bounds__(kFusedThreads) void store_fused_kernel(StoreParams p) {
  constexpr int KS = D / 16;               // K-steps
  constexpr int NC = KS / kChainSteps;     // accumulation chains
  constexpr int CW = D / 32;               // column waves
  constexpr int RG = 8 / CW;               // row blocks per round
  constexpr int TV = RG * 32;              // vectors per round
  constexpr int TPV = D / 16;              // staging threads per vector
  constexpr int XP = XT == OSCAR_F32 ? 2 : 1;  // fp16 planes of x
  constexpr int NVW = TV / 8;              // vectors per wave in the quantize phase
  constexpr int E = D / 16;                // elements per lane in the quantize phase
  constexpr int YS = D + 4;                // LDS row stride of the y tile
  static_assert(KS % kChainSteps == 0 && TV * TPV == kFusedThreads, "fused tile shape");
  const oscar_store_args_v1& a = p.a;
  const int64_t hk = a.cache.num_kv_heads;
  const int64_t kv_vec = a.num_tokens * hk;
  const int64_t q_vec = a.query_rot != nullptr ? a.num_tokens * a.num_q_heads : 0;
  // this workgroup's kind and run of rounds: workgroups [0, g) take the key rounds,
  // [g, 2 g) the value rounds and the rest the query rounds (g = p.fused_kv_groups)
  const int64_t gkv = p.fused_kv_groups;
  const int64_t b = blockIdx.x;
  const int kind = b < gkv ? KIND_K : (b < 2 * gkv ? KIND_V : KIND_Q);
  const int64_t wg = kind == KIND_K ? b : (kind == KIND_V ? b - gkv : b - 2 * gkv);
  const int64_t nwg = kind == KIND_Q ? (int64_t)gridDim.x - 2 * gkv : gkv;
  const int64_t nvec = kind == KIND_Q ? q_vec : kv_vec;
  const int64_t rounds = (nvec + TV - 1) / TV;
  const int64_t per = (rounds + nwg - 1) / nwg;
  const int64_t it0 = wg * per, it1 = it0 + per < rounds ? it0 + per : rounds;
  const int which = kind == KIND_V ? 1 : 0;  // R_v for values, R_k for keys and queries
  const void* src = kind == KIND_K ? a.key : (kind == KIND_V ? a.value : a.query);
  const int64_t stride = kind == KIND_K ? a.key_stride_token
                       : (kind == KIND_V ? a.value_stride_token : a.query_stride_token);
  void* rot_out = kind == KIND_K ? a.key_rot : (kind == KIND_V ? a.value_rot : a.query_rot);
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  const int64_t epoch = a.epoch_counter[1];
  const bool clipped = (kind == KIND_K ? a.k_clip_ratio : a.v_clip_ratio) > 0.f;  // this workgroup's kind

  const int tid = threadIdx.x, lane = tid & 63, m = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cb = wave % CW, rg = wave / CW;  // this wave's column block and row block
  const int col = 32 * cb + m;               // this lane's output column

  __shared__ u32x4 s_a[XP][RG][KS][64];      // A fragments (fp16), MFMA lane order
  // y tile, norms and destinations by round parity (one round is quantized while the
  // next one's y is formed)
  __shared__ __attribute__((aligned(16))) float s_y[2][TV][YS];
  __shared__ int s_ax[TV];                   // per-vector exponent of x
  __shared__ float s_nx[2][TV];              // ||x||
  __shared__ __attribute__((aligned(16))) float s_cn[D];  // ||R_:d||
  __shared__ Dest s_dest[2][TV];
  __shared__ int s_xn;                       // vectors this workgroup left to the exact pass
  if (tid == 0) s_xn = 0;

  // every load below is issued unconditionally (indexes clamped into range, results
  // masked at use), so the waits before their uses count exactly the loads issued since
  const int sv = tid / TPV, sq = tid % TPV;  // staging: vector, 16-element chunk
  // vector indexes fit in 31 bits (checked on the host): division by the call's fixed
  // head counts
  const FastDiv& dh = kind == KIND_Q ? p.div_hq : p.div_hk;
  auto load_x = [&](int64_t it, XChunk<XT>& xc) {
    const int64_t vec = it * TV + sv;
    const uint32_t vc = (uint32_t)(vec < nvec ? vec : nvec - 1), t = fdiv(vc, dh);
    xc.load(src, (int64_t)t * stride + (int64_t)(vc - t * dh.d) * D + 16 * sq);
  };
  // destination inputs of vector tid (< TV) of a K / V round, loaded one round ahead:
  // slot and window flag; the claims follow at the start of the round
  long long slot_n = -1;
  int32_t flag_n = 0;
  auto load_slot = [&](int64_t it) {
    const int64_t vec = it * TV + tid;
    const uint32_t t = (tid < TV && vec < kv_vec) ? fdiv((uint32_t)vec, p.div_hk) : 0u;
    slot_n = a.slot_mapping[t];
    if (window) flag_n = p.flags[t];
  };

  // ---- B: R's 32-column block in registers, the two fp16 planes written by the prep
  // kernel (lane (n, g) of K-step s: R[16 s + 8 g + j][col] * 2^bcol, j < 8), issued after
  // the first round's x so that staging does not wait for it
  const float cn = p.colnorm[which * D + col];
  const int bcol = p.bexp[which * D + col];
  XChunk<XT> xc;
  // the residual plane of the last KL K-steps is kept in LDS (each wave its own copy),
  // the rest of B in registers
  constexpr int KL = XP == 2 ? KS / 4 : KS / 2;
  __shared__ u32x4 s_b1[8][KL][64];
  u32x4 b0[KS], b1[KS - KL];
  if (it0 < it1) {
    load_x(it0, xc);
    if (kind != KIND_Q) load_slot(it0);
    const u32x4* bsrc = p.planes + ((int64_t)(which * CW + cb) * KS) * 2 * 64 + lane;
    u32x4 bl[KL];
#pragma unroll
    for (int s = 0; s < KL; ++s) bl[s] = bsrc[(2 * (KS - KL + s) + 1) * 64];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      b0[s] = bsrc[(2 * s) * 64];
      if (s < KS - KL) b1[s] = bsrc[(2 * s + 1) * 64];
    }
#pragma unroll
    for (int s = 0; s < KL; ++s) s_b1[wave][s][lane] = bl[s];
  }
  if (rg == 0 && g == 0) s_cn[col] = cn;
  float cx = 0.f;  // the rotation term of the certification bound per unit ||x|| (first round)
  int32_t* xlist = exact_list(p, kind == KIND_V ? 1 : 0, kv_vec) + it0 * TV;  // K / V: this run's segment

  // Rounds in a two-stage pipeline: each pass of the loop stages round it's x, then forms
  // round it's y~ (MFMA) and quantizes round it - 1.  The two waves that share a SIMD
  // (w and w + 4) take these two in opposite orders, so one wave's MFMAs run beside the
  // other's VALU work.
  const bool mfma_first = (wave & 4) == 0;
  static_assert(TV <= 4 * 64, "the destination threads form before they quantize");
  for (int64_t it = it0; it <= it1 && it0 < it1; ++it) {
    const bool mf = it < it1, qu = it > it0;  // this pass forms round it / quantizes it - 1
    const int cur = (int)(it & 1), prv = cur ^ 1;
    const int64_t base = it * TV;
    long long slot = -1, c_slot = -1, c_seat = -1;
    int32_t flag = 0;
    int64_t seat = 0;
    if (mf) {
      // ---- stage x: exponent, norm, fp16 planes in MFMA A order
      float f[16];
      xc.to_float(f);
      // the last round's vectors past the end stage zeros (rounds that end inside the
      // call skip the test: workgroup-uniform)
      if (base + TV > nvec && base + sv >= nvec) {
#pragma unroll
        for (int j = 0; j < 16; ++j) f[j] = 0.f;
      }
      float mx = 0.f, ss = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        mx = fmaxf(mx, fabsf(f[j]));
        ss = fmaf(f[j], f[j], ss);
      }
      mx = group_max<TPV>(mx);
      ss = group_sum<TPV>(ss);
      const int ax = fp16_exponent(mx);
      const int rb = sv / 32, mm = sv % 32;
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // chunk 2 sq + h: K-step sq, lane half h
        u32x4 w0, w1;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float h0 = ldexpf(f[8 * h + 2 * w], ax), h1 = ldexpf(f[8 * h + 2 * w + 1], ax);
          const float q0 = f16_bits_to_f32(f32_to_f16_bits(h0)), q1 = f16_bits_to_f32(f32_to_f16_bits(h1));
          w0[w] = f16_pair(q0, q1);
          w1[w] = f16_pair(h0 - q0, h1 - q1);
        }
        s_a[0][rb][sq][mm + 32 * h] = w0;
        if constexpr (XP == 2) s_a[XP - 1][rb][sq][mm + 32 * h] = w1;
      }
      if (sq == 0) {
        s_ax[sv] = ax;
        s_nx[cur][sv] = sqrtf(ss);
      }
      // ---- this round's claims (in flight until the destinations at the end of the pass)
      if (kind != KIND_Q) {
        slot = (tid < TV && base + tid < kv_vec) ? slot_n : -1;
        flag = flag_n;
        const int64_t cs = slot >= 0 && slot < p.capacity ? slot : 0;
        c_slot = (long long)a.slot_claims[cs];
        if (a.stage_mode != OSCAR_STAGE_NONE) seat = seat_of(p, cs);
        if (window) c_seat = (long long)a.seat_claims[seat];
      }
    }
    __syncthreads();
    if (it == it0) {
      // coef (1 + 2^-10)^2 max_d ||R_:d|| (the factors cover the fp32 roundings of the norms)
      float cnm = 0.f;
      for (int c = lane; c < D; c += 64) cnm = fmaxf(cnm, s_cn[c]);
      cx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(
          (XT == OSCAR_F32 ? 0x1p-19f : 0x1p-20f) * (1.f + 0x1p-10f) * (1.f + 0x1p-10f) * wave_max(cnm))));
    }
    if (mf) {  // next round's x and slots, in flight until the next pass (the last round
               // reloads its own: unconditional, so the waits count exactly)
      const int64_t nx = it + 1 < it1 ? it + 1 : it;
      load_x(nx, xc);
      if (kind != KIND_Q) load_slot(nx);
    }

    // ---- round it's destinations, for its quantize pass in the next pass of the loop
    auto dest_pass = [&]() {
      if (kind != KIND_Q && tid < TV) {
        Dest d{};
        if (slot >= 0 && slot < p.capacity) {
          const uint32_t t = fdiv((uint32_t)(base + tid), p.div_hk);
          const long long mine = claim_value(epoch, t);
          d.slot = slot;
          d.seat = seat;
          d.valid = true;
          d.slot_win = c_slot == mine;
          d.seat_win = window && c_seat == mine;
          d.keep = window && (flag & 1);
          const int64_t h = (uint32_t)(base + tid) - t * p.div_hk.d, blk = block_of(p, slot),
                        off = slot - blk * a.cache.block_size;
          d.koff = blk * a.cache.k_stride[0] + off * a.cache.k_stride[1] + h * a.cache.k_stride[2];
          d.voff = blk * a.cache.v_stride[0] + off * a.cache.v_stride[1] + h * a.cache.v_stride[2];
        }
        s_dest[cur][tid] = d;
      }
    };
    auto mfma_pass = [&]() {
      // ---- MFMA: y~ of this wave's row block x column block into the y tile.  Chains
      // of kChainSteps K-steps, each added to the running sum in fp32 as it completes
      // (each addition errs by <= 2^-24 sum_k |x_k R_kd|); the residual plane's products
      // go to their own accumulator, added last.
      f32x16 total = f32x16{}, small = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        f32x16 chain = f32x16{};
#pragma unroll
        for (int k = 0; k < kChainSteps; ++k) {
          const int s = c * kChainSteps + k;
          const f16x8 a0 = __builtin_bit_cast(f16x8, s_a[0][rg][s][lane]);
          const f16x8 f0 = __builtin_bit_cast(f16x8, b0[s]);
          const f16x8 f1 = __builtin_bit_cast(f16x8, s < KS - KL ? b1[s < KS - KL ? s : 0] : s_b1[wave][s - (KS - KL)][lane]);
          chain = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, f0, chain, 0, 0, 0);
          small = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, f1, small, 0, 0, 0);
          if constexpr (XP == 2) {
            const f16x8 a1 = __builtin_bit_cast(f16x8, s_a[1][rg][s][lane]);
            small = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, f0, small, 0, 0, 0);
            small = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, f1, small, 0, 0, 0);
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) total[r] = c == 0 ? chain[r] : total[r] + chain[r];
        // keep the A fragments' LDS reads with their chain (bounds the registers they take)
        __builtin_amdgcn_sched_barrier(0);
      }
      // C[i][n]: vector i = 8 (r / 4) + 4 g + r % 4 of the row block, column n = m
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int v = 32 * rg + 8 * (r >> 2) + 4 * g + (r & 3);
        s_y[cur][v][col] = ldexpf(total[r] + small[r], -(s_ax[v] + bcol));
      }
    };
    auto quant_pass = [&]() {
      // ---- round it - 1, four vectors at a time (one per 16-lane row, lane l holding
      // elements [l E, (l + 1) E)): read-path copy, destination, certification,
      // quantization
      const int64_t qbase = base - TV;
      const int row = lane >> 4, l = lane & 15;
#pragma unroll 1
      for (int j = 0; j < NVW / 4; ++j) {
        const int v = wave * NVW + 4 * j + row;
        const int64_t vec = qbase + v;
        const bool live = vec < nvec;
        float y[E];
#pragma unroll
        for (int q = 0; q < E; q += 4) *(f32x4*)&y[q] = *(const f32x4*)&s_y[prv][v][l * E + q];
        if (live && rot_out != nullptr) {
#pragma unroll
          for (int q = 0; q < E; q += 4) store4<XT>(rot_out, vec * D + l * E + q, &y[q]);
        }
        if (kind == KIND_Q) continue;
        Dest d{};
        if (live) d = s_dest[prv][v];
        // the slot's bytes: certified from y~, or left to the exact pass
        bool exact = false;
        if (d.valid && d.slot_win) {
          const float ex = fmaf(cx, s_nx[prv][v], 0x1p-126f);
          exact = !(clipped ? certify_quant16<D, true>(p, kind, y, ex, true, a.cache.k + d.koff, a.cache.v + d.voff)
                            : certify_quant16<D, false>(p, kind, y, ex, true, a.cache.k + d.koff, a.cache.v + d.voff));
        }
        if (exact && l == 0) xlist[atomicAdd(&s_xn, 1)] = (int32_t)vec;
        // the seat (an exact-pass vector's is written there, from y): a token in the window
        // keeps its FP32 copy -- y~ itself, within the rotation bound e of y (the bytes are
        // exact either way) -- and tags its block; a seat it wins outside the window loses
        // its FP32 copy (backend.py:513-555)
        if (d.valid && !exact && d.seat_win) {
          if (d.keep) {
            float* dst = (kind == KIND_K ? a.staging.stage_k : a.staging.stage_v) +
                         (d.seat * hk + (int64_t)fmod((uint32_t)vec, p.div_hk)) * D + l * E;
#pragma unroll
            for (int q = 0; q < E; q += 4) *(f32x4*)&dst[q] = *(const f32x4*)&y[q];
          }
          if (kind == KIND_K && l == 0) a.staging.owner[d.seat] = d.keep ? block_of(p, d.slot) : -1;
        }
      }
    };
    // the claims are only needed by waves that form before they quantize (tid < TV)
    if (mfma_first && mf) {
      mfma_pass();
      dest_pass();
    }
    if (qu) quant_pass();
    if (!mfma_first && mf) mfma_pass();
    __syncthreads();
  }
  if (kind != KIND_Q && tid == 0) exact_counts(p, kind)[wg] = s_xn;
  if (b == 0 && tid == 0) a.epoch_counter[0] = epoch;
}

// ---- exact pass: groups of kExactGroup vectors of one kind.  Thread (slice, quad) sums
// x_k R_kc in fp64 for the group's vectors, the four columns c = 4 quad .. 4 quad + 3
// and the D / S rows k of its slice (each product of an input element with an fp32
// entry is exact in fp64); R's rows come straight from global memory in batches of RB,
// the next two batches in flight during a batch's products (each batch costs one L2
// round trip), x_k of the group from LDS (one broadcast address per wave).  The slices' partial sums are added in slice order, then
// rounded once to fp32.
template <int D, int XT>
__global__ __launch_bounds__(kExactThreads) void store_exact_kernel(StoreParams p) {
  constexpr int G = kExactGroup;             // vectors per group
  constexpr int NQ = D / 4;                  // column quads
  constexpr int S = kExactThreads / NQ;      // row slices
  constexpr int RS = D / S;                  // rows per slice
  constexpr int RB = RS < 4 ? RS : 4;        // rows per batch of loads
  constexpr int TV = (8 / (D / 32)) * 32;    // vectors per round of the fused kernel
  constexpr int PT = kMaxFusedGroups / kExactThreads;  // counts per thread
  static_assert(S * NQ == kExactThreads && RS * S == D && RS % RB == 0 && G % 2 == 0, "exact tile shape");
  static_assert(PT * kExactThreads == kMaxFusedGroups && G <= 64, "counts per thread");
  const oscar_store_args_v1& a = p.a;
  const int kind = blockIdx.y;
  const int64_t hk = a.cache.num_kv_heads;
  const int64_t nvec = a.num_tokens * hk;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t epoch = a.epoch_counter[1];
  const float* R = kind == KIND_V ? a.rv : a.rk;
  const void* src = kind == KIND_K ? a.key : a.value;
  const int64_t stride = kind == KIND_K ? a.key_stride_token : a.value_stride_token;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  const int cq = tid % NQ, sl = tid / NQ;    // column quad, row slice
  const int k0 = sl * RS;
  // R[k][4 cq ..], k = k0 + kb + j; the identity for a NULL R (IDENT, a separate copy of
  // the group loop, so the loads carry no branch that would make the compiler wait)
  auto load_rows = [&](auto ident, int kb, f32x4* r) {
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int k = k0 + kb + j, o = k - 4 * cq;
      if constexpr (decltype(ident)::value)
        r[j] = f32x4{o == 0 ? 1.f : 0.f, o == 1 ? 1.f : 0.f, o == 2 ? 1.f : 0.f, o == 3 ? 1.f : 0.f};
      else
        r[j] = *(const f32x4*)(R + (int64_t)k * D + 4 * cq);
    }
  };

  // ---- the fused workgroups' counts: this thread's PT consecutive workgroups w and the
  // exclusive prefix pre[w] of all counts before them (a wave scan, then the waves)
  const int gkv = p.fused_kv_groups;
  const int64_t seg = ((nvec + TV - 1) / TV + gkv - 1) / gkv * TV;  // list entries per workgroup
  int cnt[PT], tsum = 0;
#pragma unroll
  for (int i = 0; i < PT; ++i) {
    const int w = PT * tid + i;
    cnt[i] = w < gkv ? exact_counts(p, kind)[w] : 0;
    tsum += cnt[i];
  }
  int incl = tsum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int up = __shfl_up(incl, o);
    if (lane >= o) incl += up;
  }
  __shared__ int s_wsum[kExactThreads / 64];
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  int before = incl - tsum, count = 0;
#pragma unroll
  for (int i = 0; i < kExactThreads / 64; ++i) {
    const int ws = s_wsum[i];
    if (i < wave) before += ws;
    count += ws;
  }
  if (blockIdx.x == 0 && tid == 0) p.exact[kind] = count;
  const int32_t* list = exact_list(p, kind, nvec);

  __shared__ __attribute__((aligned(16))) double s_xd[D][G];  // x_k of the group, k-major
  // the slices' partial sums: [slice][vector][column pair half][quad], one double2 each
  // (consecutive quads in consecutive 16-byte words)
  __shared__ __attribute__((aligned(16))) double2 s_part[S][G][2][NQ];
  // y of the group's vectors, rounded to fp32
  __shared__ __attribute__((aligned(16))) float s_y[G][D];
  __shared__ int32_t s_id[G];
  __shared__ int64_t s_src[G];               // element offset of each vector in the input
  __shared__ Dest s_dst[G];
  // group size: the fewest vectors (even, at most G) that give every workgroup at most
  // one group when the grid allows, so the products shrink with the count
  const int per_wg = (int)((count + gridDim.x - 1) / gridDim.x);
  const int ge = __builtin_amdgcn_readfirstlane(per_wg > G - 2 ? G : (per_wg <= 2 ? 2 : (per_wg + 1) & ~1));
  auto group_loop = [&](auto ident) {
  for (int g0 = blockIdx.x * ge; g0 < count; g0 += gridDim.x * ge) {
    // R's batches 0 (ra) and 1 (rb1), independent of the group: in flight during the
    // list reads and the staging; batch b + 2 is issued when batch b's products start
    f32x4 ra[RB], rb1[RB];
    load_rows(ident, 0, ra);
    if (RB < RS) load_rows(ident, RB, rb1);
    // ---- the group's entries: each list position g0 .. g0 + ge - 1 below count lies in
    // exactly one workgroup's segment; the thread owning that workgroup fills it (all of
    // its reads issued before the first is used: one round trip)
    {
      int32_t at[G];  // list index of group position j (below nvec), or -1 where another thread has it
      int32_t e[G];
#pragma unroll
      for (int j = 0; j < G; ++j) at[j] = -1;
      int pre = before;
#pragma unroll
      for (int i = 0; i < PT; ++i) {
#pragma unroll
        for (int j = 0; j < G; ++j)
          if (j < ge && g0 + j >= pre && g0 + j < pre + cnt[i])
            at[j] = (int32_t)((PT * tid + i) * seg + (g0 + j - pre));
        pre += cnt[i];
      }
#pragma unroll
      for (int j = 0; j < G; ++j)
        if (at[j] >= 0) e[j] = list[at[j]];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (at[j] >= 0) {
          const uint32_t id = (uint32_t)e[j];
          s_id[j] = (int32_t)id;
          s_src[j] = (int64_t)fdiv(id, p.div_hk) * stride + (int64_t)fmod(id, p.div_hk) * D;
        }
      }
      if (tid < G && (tid >= ge || g0 + tid >= count)) {
        s_id[tid] = -1;
        s_src[tid] = -1;
      }
    }
    __syncthreads();
    // destination inputs of vector tid < G: slot and window flag now, the claims after
    // the staging (in flight during the products).  Every thread reads them (token 0
    // where it has no vector), with no branch: nothing then waits for these reads
    // before the staging's reads go out.
    const int32_t d_id = tid < G ? s_id[tid] : -1;
    const int64_t d_t = fdiv((uint32_t)(d_id >= 0 ? d_id : 0), p.div_hk);
    const int64_t d_slot_in = a.slot_mapping[d_t];
    const int32_t d_flag = p.flags[d_t];
    {  // x of the group: every element's read issued before the first is used (the
       // entries past count read element k of vector 0, masked)
      constexpr int NI = G * D / kExactThreads;
      static_assert(NI * kExactThreads == G * D, "exact staging shape");
      float xs[NI];
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        const int i = tid + r * kExactThreads, v = i / D, k = i % D;
        const int64_t off = s_src[v];
        xs[r] = load_elem(src, XT, (off >= 0 ? off : 0) + k);
      }
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        const int i = tid + r * kExactThreads, v = i / D, k = i % D;
        s_xd[k][v] = s_src[v] >= 0 ? (double)xs[r] : 0.0;
      }
    }
    __syncthreads();
    long long d_cs = -1, d_cseat = -1;
    int64_t d_seat = 0;
    const int64_t d_slot = d_id >= 0 ? d_slot_in : -1;
    const bool d_valid = d_slot >= 0 && d_slot < p.capacity;
    if (tid < G && d_valid) {
      d_cs = (long long)a.slot_claims[d_slot];
      if (a.stage_mode != OSCAR_STAGE_NONE) d_seat = seat_of(p, d_slot);
      if (window) d_cseat = (long long)a.seat_claims[d_seat];
    }
    // the products of the group's first GE vectors (the group size, a multiple of 2)
    auto products = [&](auto ge_c) {
      constexpr int GE = decltype(ge_c)::value;
      double acc[GE][4];
#pragma unroll
      for (int v = 0; v < GE; ++v) acc[v][0] = acc[v][1] = acc[v][2] = acc[v][3] = 0.0;
      // batches by parity in two fixed register sets (ra: even, rb1: odd), each refilled
      // two batches ahead as soon as its products are issued, unconditionally (the last
      // two refills re-read the last batch, just fetched): no register copies and no
      // merges of loaded and unloaded values, so the waits count exactly
      auto batch = [&](int b, const f32x4* r) {
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          const int k = k0 + b * RB + j;
          const double r0 = r[j][0], r1 = r[j][1], r2 = r[j][2], r3 = r[j][3];
#pragma unroll
          for (int v = 0; v < GE; v += 2) {
            const double2 xv = *(const double2*)&s_xd[k][v];
            acc[v][0] = fma(xv.x, r0, acc[v][0]);
            acc[v][1] = fma(xv.x, r1, acc[v][1]);
            acc[v][2] = fma(xv.x, r2, acc[v][2]);
            acc[v][3] = fma(xv.x, r3, acc[v][3]);
            acc[v + 1][0] = fma(xv.y, r0, acc[v + 1][0]);
            acc[v + 1][1] = fma(xv.y, r1, acc[v + 1][1]);
            acc[v + 1][2] = fma(xv.y, r2, acc[v + 1][2]);
            acc[v + 1][3] = fma(xv.y, r3, acc[v + 1][3]);
          }
        }
      };
      constexpr int NB = RS / RB;  // batches
      static_assert(NB == 1 || NB % 2 == 0, "batches in pairs");
      if constexpr (NB == 1) {
        batch(0, ra);
      } else {
#pragma unroll 1
        for (int b = 0; b < NB; b += 2) {
          batch(b, ra);
          load_rows(ident, (b + 2 < NB ? b + 2 : NB - 1) * RB, ra);
          __builtin_amdgcn_sched_barrier(0);  // the refill stays ahead of the odd batch
          batch(b + 1, rb1);
          load_rows(ident, (b + 3 < NB ? b + 3 : NB - 1) * RB, rb1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int v = 0; v < GE; ++v) {
        s_part[sl][v][0][cq] = double2{acc[v][0], acc[v][1]};
        s_part[sl][v][1][cq] = double2{acc[v][2], acc[v][3]};
      }
    };
    static_assert(G == 8, "group sizes 2, 4, 6, 8");
    if (ge > 6) products(std::integral_constant<int, 8>{});
    else if (ge > 4) products(std::integral_constant<int, 6>{});
    else if (ge > 2) products(std::integral_constant<int, 4>{});
    else products(std::integral_constant<int, 2>{});
    if (tid < G) {  // the destination of vector tid, from its claims
      Dest d{};
      d.slot = d_slot;
      d.valid = d_valid;
      if (d_valid) {
        const long long mine = claim_value(epoch, d_t);
        d.seat = d_seat;
        d.slot_win = d_cs == mine;
        d.seat_win = window && d_cseat == mine;
        d.keep = window && (d_flag & 1);
      }
      s_dst[tid] = d;
    }
    __syncthreads();
    for (int i = tid; i < G * NQ; i += kExactThreads) {  // four columns of one vector each
      const int v = i / NQ, q = i % NQ;
      if (v >= ge) continue;
      double y0 = 0.0, y1 = 0.0, y2 = 0.0, y3 = 0.0;
#pragma unroll 4
      for (int s = 0; s < S; ++s) {
        const double2 q0 = s_part[s][v][0][q];
        const double2 q1 = s_part[s][v][1][q];
        y0 += q0.x;
        y1 += q0.y;
        y2 += q1.x;
        y3 += q1.y;
      }
      *(f32x4*)&s_y[v][4 * q] = f32x4{(float)y0, (float)y1, (float)y2, (float)y3};
    }
    __syncthreads();
    for (int v = wave; v < G; v += kExactThreads / 64) {
      const int32_t id = s_id[v];
      if (id < 0) continue;
      const f32x4 y4 = *(const f32x4*)&s_y[v][4 * (lane < D / 4 ? lane : 0)];
      quant_vector<D>(p, kind, fdiv((uint32_t)id, p.div_hk), fmod((uint32_t)id, p.div_hk), s_dst[v], y4);
    }
    __syncthreads();  // s_id, s_xd, s_part, s_y, s_dst are rewritten by the next group
  }
  };
  if (R != nullptr) group_loop(std::false_type{});
  else group_loop(std::true_type{});
}

template <int D, int XT>
int launch_large(const StoreParams& p, int cu_count, hipStream_t s) {
  constexpr int TV = (8 / (D / 32)) * 32;
  const oscar_store_args_v1& a = p.a;
  const int64_t kv_vec = a.num_tokens * a.cache.num_kv_heads;
  const int64_t q_vec = a.query_rot != nullptr ? a.num_tokens * a.num_q_heads : 0;
  const int64_t total = 2 * ((kv_vec + TV - 1) / TV) + (q_vec + TV - 1) / TV;
  const int64_t prep_blocks = (a.num_tokens + 255) / 256 + 2 * (D / 32);
  hipLaunchKernelGGL((store_prep_kernel<D>), dim3((unsigned)prep_blocks), dim3(256), 0, s, p);
  OSCAR_CHECK_LAUNCH("store_prep_kernel");
  // one workgroup per compute unit, each over a run of consecutive rounds of one kind:
  // the query rounds get their share of the workgroups, K and V the rest in halves
  const int64_t rq = (q_vec + TV - 1) / TV;
  int64_t grid = total < cu_count ? total : cu_count;
  if (grid > 2 * kMaxFusedGroups) grid = 2 * kMaxFusedGroups;
  if (grid < (rq > 0 ? 3 : 2)) grid = rq > 0 ? 3 : 2;
  int64_t gq = 0;
  if (rq > 0) {
    gq = grid * rq / total;
    if (gq < 1) gq = 1;
    if (gq > grid - 2) gq = grid - 2;
  }
  StoreParams q = p;
  q.fused_kv_groups = (int32_t)((grid - gq) / 2);
  grid = 2 * q.fused_kv_groups + gq;
  hipLaunchKernelGGL((store_fused_kernel<D, XT>), dim3((unsigned)grid), dim3(kFusedThreads), 0, s, q);
  OSCAR_CHECK_LAUNCH("store_fused_kernel");
  // persistent over the device-side counts: per kind at most half the compute units
  // (the list is a few percent of the vectors plus the window's)
  int64_t groups = (kv_vec + kExactGroup - 1) / kExactGroup;
  const int64_t half_cus = cu_count / 2 > 0 ? cu_count / 2 : 1;
  if (groups > half_cus) groups = half_cus;
  hipLaunchKernelGGL((store_exact_kernel<D, XT>), dim3((unsigned)groups, 2), dim3(kExactThreads), 0, s, q);
  OSCAR_CHECK_LAUNCH("store_exact_kernel");
  return 0;
}

template <int D>
int launch_store(const StoreParams& p, int cu_count, hipStream_t s) {
  const int XT = p.a.kv_dtype;
  if (p.a.num_tokens <= kFusedTokens) {
    const int64_t hk = p.a.cache.num_kv_heads;
    const int64_t qg = p.a.query_rot != nullptr ? small_groups(p.a.num_tokens * p.a.num_q_heads) : 0;
    dim3 grid((unsigned)(D / kSmallCols), (unsigned)(2 * small_groups(p.a.num_tokens * hk) + qg));
    if (XT == OSCAR_BF16) hipLaunchKernelGGL((store_small_kernel<D, OSCAR_BF16>), grid, dim3(kSmallThreads), 0, s, p);
    else if (XT == OSCAR_F16) hipLaunchKernelGGL((store_small_kernel<D, OSCAR_F16>), grid, dim3(kSmallThreads), 0, s, p);
    else hipLaunchKernelGGL((store_small_kernel<D, OSCAR_F32>), grid, dim3(kSmallThreads), 0, s, p);
    OSCAR_CHECK_LAUNCH("store_small_kernel");
    return 0;
  }
  if (XT == OSCAR_BF16) return launch_large<D, OSCAR_BF16>(p, cu_count, s);
  if (XT == OSCAR_F16) return launch_large<D, OSCAR_F16>(p, cu_count, s);
  return launch_large<D, OSCAR_F32>(p, cu_count, s);
}

}  // namespace

}  // namespace oscar

using namespace oscar;

// workspace: calls of <= kFusedTokens tokens: y [2][N][Hk][D] fp32 (the column slices);
// larger calls: the exact-pass totals, per-workgroup counts and lists
// (2 + 2 kMaxFusedGroups + 2 N Hk int32) | window flags [N] int32
static int64_t store_ws_list_bytes(int64_t n, int64_t hk) {
  return ((2 + 2 * kMaxFusedGroups + 2 * n * hk) * (int64_t)sizeof(int32_t) + 15) / 16 * 16;
}

static int64_t store_ws_flag_bytes(int64_t n) { return (n * (int64_t)sizeof(int32_t) + 15) / 16 * 16; }
// fp16 planes of R_k and R_v (2 x D x D x 2 planes x 2 bytes), then bexp and colnorm [2][D] each
static int64_t store_ws_plane_bytes(int64_t d) { return 8 * d * d + 16 * d; }

extern "C" int64_t oscar_store_workspace_bytes_v1(int64_t num_tokens, int64_t num_kv_heads,
                                                 int64_t head_dim) {
  if (num_tokens <= kFusedTokens) return 2 * num_tokens * num_kv_heads * head_dim * (int64_t)sizeof(float);
  return store_ws_list_bytes(num_tokens, num_kv_heads) + store_ws_flag_bytes(num_tokens) +
         store_ws_plane_bytes(head_dim);
}

// compute units of the current device (cached per device)
static int current_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cu = cache[dev].load(std::memory_order_relaxed);
  if (cu <= 0) {
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
    cache[dev].store(cu, std::memory_order_relaxed);
  }
  return cu;
}

int oscar::store_launch(const oscar_store_args_v1* args, void* stream, bool defer, const char* fn, StoreParams* out) {
  *out = StoreParams{};
  if (args == nullptr) return fail(-22, "%s: null args", fn);
  const oscar_store_args_v1& a = *args;
  if (a.num_tokens < 0) return fail(-22, "%s: negative num_tokens", fn);
  if (a.num_tokens == 0) return 0;
  const int64_t D = a.cache.head_dim;
  if (D != 64 && D != 128 && D != 256)
    return fail(-22, "%s: head_dim %lld unsupported (64/128/256)", fn, (long long)D);
  if (a.key == nullptr || a.value == nullptr || a.slot_mapping == nullptr)
    return fail(-22, "%s: key/value/slot_mapping required", fn);
  if (a.kv_dtype != OSCAR_BF16 && a.kv_dtype != OSCAR_F16 && a.kv_dtype != OSCAR_F32)
    return fail(-22, "%s: bad kv_dtype %d", fn, a.kv_dtype);
  if (a.cache.k == nullptr || a.cache.v == nullptr || a.cache.block_size <= 0 ||
      a.cache.num_blocks <= 0 || a.cache.num_kv_heads <= 0)
    return fail(-22, "%s: invalid cache geometry", fn);
  if (a.cache.k_stride[2] < 32 + D / 4 || a.cache.v_stride[2] < D / 4)
    return fail(-22, "%s: slot stride too small for the packed layout", fn);
  for (int i = 0; i < 3; ++i)
    if ((a.cache.k_stride[i] & 3) || (a.cache.v_stride[i] & 3))
      return fail(-22, "%s: cache strides must be multiples of 4 bytes", fn);
  if ((((uintptr_t)a.cache.k) & 3) || (((uintptr_t)a.cache.v) & 3))
    return fail(-22, "%s: cache base must be 4-byte aligned", fn);
  if (a.key_stride_token < a.cache.num_kv_heads * D || a.value_stride_token < a.cache.num_kv_heads * D)
    return fail(-22, "%s: key/value row stride smaller than heads*D", fn);
  // inputs are read 8 elements (16 or 32 bytes) at a time, outputs written 4 at a time
  const int esz = a.kv_dtype == OSCAR_F32 ? 4 : 2;
  auto misaligned = [&](const void* ptr, int64_t stride) {
    return ptr != nullptr && ((((uintptr_t)ptr) & 15) || ((stride * esz) & 15));
  };
  if (misaligned(a.key, a.key_stride_token) || misaligned(a.value, a.value_stride_token) ||
      (a.query_rot != nullptr && misaligned(a.query, a.query_stride_token)))
    return fail(-22, "%s: key/value/query rows must be 16-byte aligned", fn);
  if ((a.key_rot && (((uintptr_t)a.key_rot) & 15)) || (a.value_rot && (((uintptr_t)a.value_rot) & 15)) ||
      (a.query_rot && (((uintptr_t)a.query_rot) & 15)))
    return fail(-22, "%s: rotated outputs must be 16-byte aligned", fn);
  if ((a.rk && (((uintptr_t)a.rk) & 15)) || (a.rv && (((uintptr_t)a.rv) & 15)))
    return fail(-22, "%s: rotations must be 16-byte aligned", fn);
  if (a.slot_claims == nullptr || a.epoch_counter == nullptr)
    return fail(-22, "%s: slot_claims scratch and the device epoch counter are required", fn);
  if (a.num_tokens >= (1ll << 24)) return fail(-22, "%s: more than 2^24 tokens per call", fn);
  if (a.stage_mode != OSCAR_STAGE_NONE) {
    if (a.staging.owner == nullptr || a.staging.rows <= 0)
      return fail(-22, "%s: staging arena required for stage_mode %d", fn, a.stage_mode);
    if (a.stage_mode == OSCAR_STAGE_WRITE &&
        (a.seat_claims == nullptr || a.staging.stage_k == nullptr || a.staging.stage_v == nullptr ||
         a.query_start_loc == nullptr || a.seq_lens == nullptr || a.num_reqs <= 0))
      return fail(-22, "%s: window write needs seat_claims, arena and request metadata", fn);
    if (a.stage_mode == OSCAR_STAGE_WRITE &&
        ((((uintptr_t)a.staging.stage_k) & 15) || (((uintptr_t)a.staging.stage_v) & 15)))
      return fail(-22, "%s: staging arena must be 16-byte aligned", fn);
  }
  if (a.query_rot != nullptr &&
      (a.query == nullptr || a.num_q_heads <= 0 || a.query_stride_token < a.num_q_heads * D))
    return fail(-22, "%s: query_rot requires query, num_q_heads and a valid stride", fn);
  const int64_t need = oscar_store_workspace_bytes_v1(a.num_tokens, a.cache.num_kv_heads, D);
  if (a.workspace == nullptr || a.workspace_bytes < need || (((uintptr_t)a.workspace) & 15))
    return fail(-22, "%s: 16-byte aligned workspace of %lld bytes required", fn, (long long)need);
  if (a.num_tokens <= kFusedTokens && (a.arrivals == nullptr || (((uintptr_t)a.arrivals) & 3)))
    return fail(-22, "%s: calls of <= %lld tokens need the arrivals counters", fn, (long long)kFusedTokens);
  if (2 * a.num_tokens * a.cache.num_kv_heads >= (1ll << 31) ||
      (a.query_rot != nullptr && a.num_tokens * a.num_q_heads >= (1ll << 31)))
    return fail(-22, "%s: num_tokens x heads too large for one call", fn);
  StoreParams p{a, (float*)a.workspace, a.cache.num_blocks * a.cache.block_size};
  p.slots31 = p.capacity < (1ll << 31);
  p.div_hk = FastDiv::of(a.cache.num_kv_heads);
  p.div_hq = FastDiv::of(a.num_q_heads);
  p.div_bs = FastDiv::of(a.cache.block_size);
  p.div_rows = FastDiv::of(a.staging.rows);
  uint8_t* ws = (uint8_t*)a.workspace;
  p.exact = (int32_t*)ws;
  p.flags = (int32_t*)(ws + store_ws_list_bytes(a.num_tokens, a.cache.num_kv_heads));
  p.planes = (u32x4*)((uint8_t*)p.flags + store_ws_flag_bytes(a.num_tokens));
  p.bexp = (int32_t*)(p.planes + D * D / 2);
  p.colnorm = (float*)(p.bexp + 2 * D);
  const int cu = a.num_tokens <= kFusedTokens ? 0 : current_cu_count();
  hipStream_t s = (hipStream_t)stream;
  p.deferred = defer && a.num_tokens <= kFusedTokens;
  *out = p;
  if (D == 256) return launch_store<256>(p, cu, s);
  if (D == 128) return launch_store<128>(p, cu, s);
  return launch_store<64>(p, cu, s);
}

extern "C" int oscar_store_v1(const oscar_store_args_v1* args, void* stream) {
  StoreParams p;
  return store_launch(args, stream, false, "oscar_store_v1", &p);
}
