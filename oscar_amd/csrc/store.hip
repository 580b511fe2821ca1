// INT2 write path for gfx950: rotate, sort-clip, quantize, pack, scatter, staging.
//
// Replaces oscar_ascend/kernels/store_kernel.py:54-102 / :166-279 and the
// host-side pieces of oscar_ascend/backend.py around them (_rotate_clip
// :130-148, do_kv_cache_update :151-198, _staging_write :513-555, and the
// read-path rotations :370-373).
//
// Two launches:
//   store_rotate_kernel  grid (vector tiles, 64-column blocks, kind in {K, V, Q}).
//                        y = x @ R with fp64 accumulation: every product of a
//                        bf16/fp16/fp32 input with an fp32 rotation entry is exact in
//                        fp64 and the sum is rounded once, which yields the correctly
//                        rounded fp32 value independent of summation order.  Writes y
//                        (fp32 workspace, K/V only) and the read-path copies in the
//                        input dtype.  Column block 0 of the K kind also records the
//                        last-writer claims (64-bit atomicMax of epoch<<32 | token)
//                        for cache slots and staging seats, and performs the owner-tag
//                        invalidation of a standalone KV update.
//   store_quant_kernel   one wave per (token, kv head, K|V) vector: optional sort-clip,
//                        fp16-rounded scale/zero, codes clamp(floor((x-zero)/scale+0.5),
//                        0, 3), 2-bit packing and the byte writes of the slot winner;
//                        staging winners write the owner tag and, inside the sink/recent
//                        window, the unclipped fp32 rotated vector.
#include "common.h"

namespace oscar {

namespace {

constexpr int kThreads = 256;
constexpr int kCols = 64;     // output columns per rotate workgroup
constexpr int kChunk = 32;    // contraction rows staged in LDS per step

enum Kind { KIND_K = 0, KIND_V = 1, KIND_Q = 2 };

struct StoreParams {
  oscar_store_args_v1 a;
  float* y;          // workspace [2][num_tokens][num_kv_heads][D] fp32 (K then V)
  int64_t capacity;  // num_blocks * block_size
};

__device__ __forceinline__ long long claim_value(int64_t epoch, int64_t token) {
  // 39-bit epoch above a 24-bit token index: 5e11 calls before the counter saturates
  return (long long)((epoch << 24) | (token & 0xffffffll));
}

__device__ __forceinline__ int64_t seat_of(int64_t slot, int64_t bs, int64_t rows) {
  return ((slot / bs) % rows) * bs + slot % bs;
}

template <int D, int TV>
__global__ __launch_bounds__(kThreads) void store_rotate_kernel(StoreParams p) {
  const oscar_store_args_v1& a = p.a;
  const int kind = blockIdx.z;
  const int64_t heads = (kind == KIND_Q) ? a.num_q_heads : a.cache.num_kv_heads;
  const int64_t nvec = a.num_tokens * heads;
  const int64_t vec0 = (int64_t)blockIdx.x * TV;
  if (vec0 >= nvec) return;
  const int col0 = blockIdx.y * kCols;
  const int tid = threadIdx.x;

  // last-writer claims and standalone invalidation, once per token
  if (kind == KIND_K && blockIdx.y == 0) {
    const int64_t epoch = *a.epoch_counter + 1;
    for (int i = tid; i < TV; i += kThreads) {
      int64_t vec = vec0 + i;
      if (vec >= nvec || vec % heads != 0) continue;
      int64_t t = vec / heads;
      int64_t s = a.slot_mapping[t];
      if (s < 0 || s >= p.capacity) continue;
      atomicMax((unsigned long long*)&a.slot_claims[s], (unsigned long long)claim_value(epoch, t));
      if (a.stage_mode == OSCAR_STAGE_NONE) continue;
      int64_t seat = seat_of(s, a.cache.block_size, a.staging.rows);
      if (a.stage_mode == OSCAR_STAGE_INVALIDATE) a.staging.owner[seat] = -1;
      else atomicMax((unsigned long long*)&a.seat_claims[seat], (unsigned long long)claim_value(epoch, t));
    }
  }

  const void* src = kind == KIND_K ? a.key : (kind == KIND_V ? a.value : a.query);
  const int64_t src_stride = kind == KIND_K ? a.key_stride_token
                           : (kind == KIND_V ? a.value_stride_token : a.query_stride_token);
  const float* R = (kind == KIND_V) ? a.rv : a.rk;
  void* rot_out = kind == KIND_K ? a.key_rot : (kind == KIND_V ? a.value_rot : a.query_rot);
  float* y_out = (kind == KIND_Q) ? nullptr : p.y + (int64_t)kind * a.num_tokens * heads * D;

  __shared__ double xs[kChunk][TV];
  // thread tile: 4 consecutive columns x RPT vectors
  constexpr int kColGroups = kCols / 4;              // 16
  constexpr int kRowGroups = kThreads / kColGroups;  // 16
  constexpr int RPT = TV / kRowGroups;
  static_assert(RPT >= 1 && TV % kRowGroups == 0, "tile");
  const int cg = tid % kColGroups, rg = tid / kColGroups;
  double acc[RPT][4];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;

  for (int k0 = 0; k0 < D; k0 += kChunk) {
    __syncthreads();
    for (int e = tid; e < kChunk * TV; e += kThreads) {
      int vv = e / kChunk, kk = e % kChunk;
      int64_t vec = vec0 + vv;
      double x = 0.0;
      if (vec < nvec) {
        int64_t t = vec / heads, h = vec % heads;
        x = (double)load_elem(src, a.kv_dtype, t * src_stride + h * D + k0 + kk);
      }
      xs[kk][vv] = x;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < kChunk; ++kk) {
      double r0, r1, r2, r3;
      if (R != nullptr) {
        float4 r4 = *(const float4*)(R + (int64_t)(k0 + kk) * D + col0 + cg * 4);
        r0 = r4.x; r1 = r4.y; r2 = r4.z; r3 = r4.w;
      } else {
        int c = col0 + cg * 4 - (k0 + kk);
        r0 = c == 0; r1 = c == -1; r2 = c == -2; r3 = c == -3;
      }
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        double x = xs[kk][rg * RPT + i];
        acc[i][0] = fma(x, r0, acc[i][0]);
        acc[i][1] = fma(x, r1, acc[i][1]);
        acc[i][2] = fma(x, r2, acc[i][2]);
        acc[i][3] = fma(x, r3, acc[i][3]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    int64_t vec = vec0 + rg * RPT + i;
    if (vec >= nvec) continue;
    float y[4] = {(float)acc[i][0], (float)acc[i][1], (float)acc[i][2], (float)acc[i][3]};
    int64_t base = vec * D + col0 + cg * 4;
    if (y_out != nullptr) *(float4*)(y_out + base) = make_float4(y[0], y[1], y[2], y[3]);
    if (rot_out != nullptr) {
#pragma unroll
      for (int j = 0; j < 4; ++j) store_elem(rot_out, a.kv_dtype, base + j, y[j]);
    }
  }
}

// token -> request by binary search over query_start_loc clipped to num_tokens
__device__ int find_request(const int32_t* qsl, int num_reqs, int64_t num_tokens, int64_t t) {
  int lo = 0, hi = num_reqs;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    int64_t start = qsl[mid] < num_tokens ? qsl[mid] : num_tokens;
    if (start <= t) lo = mid; else hi = mid;
  }
  return lo;
}

// Sort-based clip threshold (backend.py:140-145): the idx-th smallest |x| of a
// D-vector stored in LDS; ties are ordered by index so exactly one lane matches.
template <int D>
__device__ float clip_threshold(const float* row, int idx, volatile float* slot) {
  const int lane = threadIdx.x & 63;
  for (int i = lane; i < D; i += 64) {
    float xi = fabsf(row[i]);
    int rank = 0;
    for (int j = 0; j < D; ++j) {
      float xj = fabsf(row[j]);
      rank += (xj < xi) || (xj == xi && j < i);
    }
    if (rank == idx) *slot = xi;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  return *slot;
}

template <int D>
__global__ __launch_bounds__(kThreads) void store_quant_kernel(StoreParams p) {
  const oscar_store_args_v1& a = p.a;
  const int kind = blockIdx.y;  // K or V
  const int64_t hk = a.cache.num_kv_heads;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t vec = (int64_t)blockIdx.x * (kThreads / 64) + wave;
  if (vec >= a.num_tokens * hk) return;
  const int64_t t = vec / hk, h = vec % hk;
  const int64_t slot = a.slot_mapping[t];
  if (slot < 0 || slot >= p.capacity) return;
  const int64_t epoch = *a.epoch_counter + 1;

  __shared__ float rows[kThreads / 64][D];
  __shared__ float clip_slot[kThreads / 64];
  float* row = rows[wave];
  const float* y = p.y + ((int64_t)kind * a.num_tokens * hk + vec) * D;
  for (int i = lane; i < D; i += 64) row[i] = y[i];
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();

  const int64_t bs = a.cache.block_size;
  const int64_t blk = slot / bs, off = slot % bs;
  if (a.stage_mode == OSCAR_STAGE_WRITE) {
    const int64_t seat = seat_of(slot, bs, a.staging.rows);
    if ((long long)a.seat_claims[seat] == claim_value(epoch, t)) {
      int r = find_request(a.query_start_loc, a.num_reqs, a.num_tokens, t);
      int64_t seq = a.seq_lens[r], end = a.query_start_loc[r + 1];
      int64_t pos = seq - end + t;
      bool keep = (pos >= seq - a.recent_tokens) || (pos < a.sink_tokens_eff);
      if (kind == KIND_K && lane == 0) a.staging.owner[seat] = keep ? blk : -1;
      if (keep) {
        float* dst = (kind == KIND_K ? a.staging.stage_k : a.staging.stage_v) + (seat * hk + h) * D;
        for (int i = lane; i < D; i += 64) dst[i] = row[i];
      }
    }
  }
  if ((long long)a.slot_claims[slot] != claim_value(epoch, t)) return;

  const float clip = kind == KIND_K ? a.k_clip_ratio : a.v_clip_ratio;
  float thr = INFINITY;
  if (clip > 0.f) {
    int idx = (int)(clip * (float)D);
    if (idx > D - 1) idx = D - 1;
    thr = clip_threshold<D>(row, idx, &clip_slot[wave]);
  }
  // lane b handles byte b = elements 4b..4b+3
  const bool active = lane < D / 4;
  float x[4];
  float vmin = INFINITY, vmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = active ? row[lane * 4 + j] : 0.f;
    if (clip > 0.f) v = fminf(fmaxf(v, -thr), thr);
    x[j] = v;
    if (active) { vmin = fminf(vmin, v); vmax = fmaxf(vmax, v); }
  }
  vmin = wave_min(vmin);
  vmax = wave_max(vmax);
  float scale = __fdiv_rn(vmax - vmin, 3.0f);
  if (!(scale > 0x1p-14f)) scale = 0x1p-14f;
  const unsigned short scale_bits = f32_to_f16_bits(scale);
  const unsigned short zero_bits = f32_to_f16_bits(vmin);
  const float s16 = f16_bits_to_f32(scale_bits), z16 = f16_bits_to_f32(zero_bits);
  uint8_t* kslot = a.cache.k + blk * a.cache.k_stride[0] + off * a.cache.k_stride[1] + h * a.cache.k_stride[2];
  uint8_t* vslot = a.cache.v + blk * a.cache.v_stride[0] + off * a.cache.v_stride[1] + h * a.cache.v_stride[2];
  if (active) {
    unsigned byte = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float q = floorf(__fdiv_rn(x[j] - z16, s16) + 0.5f);
      q = fminf(fmaxf(q, 0.f), 3.f);
      byte |= (unsigned)((int)q & 3) << (2 * j);
    }
    uint8_t* dst = (kind == KIND_K) ? (kslot + 32) : vslot;
    dst[lane] = (uint8_t)byte;
  }
  if (lane == 0) {
    unsigned meta = (unsigned)scale_bits | ((unsigned)zero_bits << 16);
    *(unsigned*)(kslot + (kind == KIND_K ? 0 : 4)) = meta;
  }
}

// Advance the per-device claim epoch once both launches of a call have finished
// (vector store: the counter is ordinary device memory).
__global__ void store_epoch_kernel(int64_t* counter) {
  const int64_t e = *counter + 1;
  if (e < (1ll << 39) - 1) *counter = e;  // saturates (5e11 calls) instead of wrapping
}

template <int D>
int launch_store(const StoreParams& p, int64_t kv_vec, int64_t q_vec, hipStream_t s) {
  const int kinds = q_vec ? 3 : 2;
  const int64_t max_vec = kv_vec > q_vec ? kv_vec : q_vec;
  dim3 block(kThreads);
  if (max_vec >= 4096) {
    dim3 grid((unsigned)((max_vec + 63) / 64), D / kCols, kinds);
    hipLaunchKernelGGL((store_rotate_kernel<D, 64>), grid, block, 0, s, p);
  } else {
    dim3 grid((unsigned)((max_vec + 15) / 16), D / kCols, kinds);
    hipLaunchKernelGGL((store_rotate_kernel<D, 16>), grid, block, 0, s, p);
  }
  OSCAR_CHECK_LAUNCH("store_rotate_kernel");
  dim3 qgrid((unsigned)((kv_vec + 3) / 4), 2);
  hipLaunchKernelGGL(store_quant_kernel<D>, qgrid, block, 0, s, p);
  OSCAR_CHECK_LAUNCH("store_quant_kernel");
  hipLaunchKernelGGL(store_epoch_kernel, dim3(1), dim3(1), 0, s, p.a.epoch_counter);
  OSCAR_CHECK_LAUNCH("store_epoch_kernel");
  return 0;
}

}  // namespace

}  // namespace oscar

using namespace oscar;

extern "C" int64_t oscar_store_workspace_bytes_v1(int64_t num_tokens, int64_t num_kv_heads,
                                                 int64_t head_dim) {
  return 2 * num_tokens * num_kv_heads * head_dim * (int64_t)sizeof(float);
}

extern "C" int oscar_store_v1(const oscar_store_args_v1* args, void* stream) {
  if (args == nullptr) return fail(-22, "oscar_store_v1: null args");
  const oscar_store_args_v1& a = *args;
  if (a.num_tokens < 0) return fail(-22, "oscar_store_v1: negative num_tokens");
  if (a.num_tokens == 0) return 0;
  const int64_t D = a.cache.head_dim;
  if (D != 64 && D != 128 && D != 256)
    return fail(-22, "oscar_store_v1: head_dim %lld unsupported (64/128/256)", (long long)D);
  if (a.key == nullptr || a.value == nullptr || a.slot_mapping == nullptr)
    return fail(-22, "oscar_store_v1: key/value/slot_mapping required");
  if (a.kv_dtype != OSCAR_BF16 && a.kv_dtype != OSCAR_F16 && a.kv_dtype != OSCAR_F32)
    return fail(-22, "oscar_store_v1: bad kv_dtype %d", a.kv_dtype);
  if (a.cache.k == nullptr || a.cache.v == nullptr || a.cache.block_size <= 0 ||
      a.cache.num_blocks <= 0 || a.cache.num_kv_heads <= 0)
    return fail(-22, "oscar_store_v1: invalid cache geometry");
  if (a.cache.k_stride[2] < 32 + D / 4 || a.cache.v_stride[2] < D / 4)
    return fail(-22, "oscar_store_v1: slot stride too small for the packed layout");
  for (int i = 0; i < 3; ++i)
    if ((a.cache.k_stride[i] & 3) || (a.cache.v_stride[i] & 3))
      return fail(-22, "oscar_store_v1: cache strides must be multiples of 4 bytes");
  if ((((uintptr_t)a.cache.k) & 3) || (((uintptr_t)a.cache.v) & 3))
    return fail(-22, "oscar_store_v1: cache base must be 4-byte aligned");
  if (a.key_stride_token < a.cache.num_kv_heads * D || a.value_stride_token < a.cache.num_kv_heads * D)
    return fail(-22, "oscar_store_v1: key/value row stride smaller than heads*D");
  if ((a.rk && (((uintptr_t)a.rk) & 15)) || (a.rv && (((uintptr_t)a.rv) & 15)))
    return fail(-22, "oscar_store_v1: rotations must be 16-byte aligned");
  if (a.slot_claims == nullptr || a.epoch_counter == nullptr)
    return fail(-22, "oscar_store_v1: slot_claims scratch and the device epoch counter are required");
  if (a.num_tokens >= (1ll << 24)) return fail(-22, "oscar_store_v1: more than 2^24 tokens per call");
  if (a.stage_mode != OSCAR_STAGE_NONE) {
    if (a.staging.owner == nullptr || a.staging.rows <= 0)
      return fail(-22, "oscar_store_v1: staging arena required for stage_mode %d", a.stage_mode);
    if (a.stage_mode == OSCAR_STAGE_WRITE &&
        (a.seat_claims == nullptr || a.staging.stage_k == nullptr || a.staging.stage_v == nullptr ||
         a.query_start_loc == nullptr || a.seq_lens == nullptr || a.num_reqs <= 0))
      return fail(-22, "oscar_store_v1: window write needs seat_claims, arena and request metadata");
  }
  if (a.query_rot != nullptr &&
      (a.query == nullptr || a.num_q_heads <= 0 || a.query_stride_token < a.num_q_heads * D))
    return fail(-22, "oscar_store_v1: query_rot requires query, num_q_heads and a valid stride");
  const int64_t need = oscar_store_workspace_bytes_v1(a.num_tokens, a.cache.num_kv_heads, D);
  if (a.workspace == nullptr || a.workspace_bytes < need || (((uintptr_t)a.workspace) & 15))
    return fail(-22, "oscar_store_v1: 16-byte aligned workspace of %lld bytes required", (long long)need);
  StoreParams p{a, (float*)a.workspace, a.cache.num_blocks * a.cache.block_size};
  const int64_t kv_vec = a.num_tokens * a.cache.num_kv_heads;
  const int64_t q_vec = (a.query_rot != nullptr) ? a.num_tokens * a.num_q_heads : 0;
  hipStream_t s = (hipStream_t)stream;
  if (D == 256) return launch_store<256>(p, kv_vec, q_vec, s);
  if (D == 128) return launch_store<128>(p, kv_vec, q_vec, s);
  return launch_store<64>(p, kv_vec, q_vec, s);
}
