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
//                        rounded fp32 value independent of summation order.  The
//                        workgroup stages its 64 columns of R and its input vectors in
//                        LDS with one batch of vector loads, then accumulates from LDS.
//                        Writes y (fp32 workspace, K/V only) and the read-path copies
//                        in the input dtype.  Column block 0 of the K kind also records
//                        the last-writer claims (64-bit atomicMax of epoch<<24 | token)
//                        for cache slots and staging seats, and performs the owner-tag
//                        invalidation of a standalone KV update.
//   store_quant_kernel   one wave per (token, kv head, K|V) vector: optional sort-clip,
//                        fp16-rounded scale/zero, codes clamp(floor((x-zero)/scale+0.5),
//                        0, 3), 2-bit packing and the byte writes of the slot winner;
//                        staging winners write the owner tag and, inside the sink/recent
//                        window, the unclipped fp32 rotated vector.  Its global reads
//                        come in two rounds (slot, row, request bounds; then the claims).
//
// Claim epochs live on the device in two int64 words so that a captured graph
// replays with fresh epochs and no extra launch: the rotate kernel uses
// E = word0 + 1 and stores E in word1; the quant kernel reads word1 and copies it
// to word0 for the next call.
#include "common.h"

namespace oscar {

namespace {

constexpr int kThreads = 256;
constexpr int kCols = 64;     // output columns per rotate workgroup

enum Kind { KIND_K = 0, KIND_V = 1, KIND_Q = 2 };

struct StoreParams {
  oscar_store_args_v1 a;
  float* y;          // workspace [2][num_tokens][num_kv_heads][D] fp32 (K then V)
  int64_t capacity;  // num_blocks * block_size
  int scan;          // small call: winners found by scanning slot_mapping (no claims)
};

// calls of at most this many tokens resolve last writers by scanning
constexpr int64_t kScanTokens = 1024;

__device__ __forceinline__ long long claim_value(int64_t epoch, int64_t token) {
  // 39-bit epoch above a 24-bit token index: 5e11 calls before the counter saturates
  return (long long)((epoch << 24) | (token & 0xffffffll));
}
constexpr int64_t kMaxEpoch = (1ll << 39) - 1;

__device__ __forceinline__ int64_t seat_of(int64_t slot, int64_t bs, int64_t rows) {
  return ((slot / bs) % rows) * bs + slot % bs;
}

// 4 floats to dtype DT at element i (8 or 16 bytes, aligned)
template <int DT>
__device__ __forceinline__ void store4(void* base, int64_t i, const float* y) {
  if constexpr (DT == OSCAR_F32) {
    *(f32x4*)((float*)base + i) = f32x4{y[0], y[1], y[2], y[3]};
  } else {
    unsigned w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const unsigned lo = DT == OSCAR_BF16 ? f32_to_bf16_bits(y[2 * j]) : f32_to_f16_bits(y[2 * j]);
      const unsigned hi = DT == OSCAR_BF16 ? f32_to_bf16_bits(y[2 * j + 1]) : f32_to_f16_bits(y[2 * j + 1]);
      w[j] = lo | (hi << 16);
    }
    *(u32x2*)((uint16_t*)base + i) = u32x2{w[0], w[1]};
  }
}

// Last-writer claims and standalone invalidation for vectors [vec0, vec0 + count)
// of the K kind (once per token: head 0); block (0, 0) publishes the call's epoch.
__device__ void record_claims(const StoreParams& p, int64_t vec0, int count, int64_t heads, int64_t nvec) {
  const oscar_store_args_v1& a = p.a;
  const int64_t e0 = a.epoch_counter[0];
  const int64_t epoch = e0 < kMaxEpoch ? e0 + 1 : kMaxEpoch;
  if (blockIdx.x == 0 && threadIdx.x == 0) a.epoch_counter[1] = epoch;
  for (int i = threadIdx.x; i < count; i += blockDim.x) {
    const int64_t vec = vec0 + i;
    if (vec >= nvec || vec % heads != 0) continue;
    const int64_t t = vec / heads;
    const int64_t s = a.slot_mapping[t];
    if (s < 0 || s >= p.capacity) continue;
    atomicMax((unsigned long long*)&a.slot_claims[s], (unsigned long long)claim_value(epoch, t));
    if (a.stage_mode == OSCAR_STAGE_NONE) continue;
    const int64_t seat = seat_of(s, a.cache.block_size, a.staging.rows);
    if (a.stage_mode == OSCAR_STAGE_INVALIDATE) a.staging.owner[seat] = -1;
    else atomicMax((unsigned long long*)&a.seat_claims[seat], (unsigned long long)claim_value(epoch, t));
  }
}

// Small calls (decode steps): 16 vectors x 16 columns per workgroup, the
// contraction split over the four waves (64-key quarters each, fp64 accumulate),
// partial sums added in wave order in LDS, so a 32-token step spreads over ~1024
// waves instead of a few long fp64 chains.
constexpr int kSV = 16, kSC = 16;

template <int D, int XT>
__global__ __launch_bounds__(kThreads) void store_rotate_small_kernel(StoreParams p) {
  const oscar_store_args_v1& a = p.a;
  const int kind = blockIdx.z;
  const int64_t heads = (kind == KIND_Q) ? a.num_q_heads : a.cache.num_kv_heads;
  const int64_t nvec = a.num_tokens * heads;
  const int64_t vec0 = (int64_t)blockIdx.x * kSV;
  if (vec0 >= nvec) return;
  const int col0 = blockIdx.y * kSC;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const void* src = kind == KIND_K ? a.key : (kind == KIND_V ? a.value : a.query);
  const int64_t src_stride = kind == KIND_K ? a.key_stride_token
                           : (kind == KIND_V ? a.value_stride_token : a.query_stride_token);
  const float* R = (kind == KIND_V) ? a.rv : a.rk;
  void* rot_out = kind == KIND_K ? a.key_rot : (kind == KIND_V ? a.value_rot : a.query_rot);
  float* y_out = (kind == KIND_Q) ? nullptr : p.y + (int64_t)kind * a.num_tokens * heads * D;

  __shared__ __attribute__((aligned(16))) float s_r[D][kSC];
  __shared__ float s_x[D][kSV + 1];
  __shared__ double s_red[3][4][64];
  constexpr int RN = D * kSC / 4;   // float4 of R
  constexpr int XN = kSV * D / 8;   // 8-element x loads
  constexpr int RI = (RN + kThreads - 1) / kThreads, XI = (XN + kThreads - 1) / kThreads;
  f32x4 rr[RI];
  float xv[XI][8];
#pragma unroll
  for (int i = 0; i < RI; ++i) {
    const int e = tid + i * kThreads, k = e / (kSC / 4), c4 = e % (kSC / 4);
    if (e >= RN) break;
    if (R != nullptr) {
      rr[i] = *(const f32x4*)(R + (int64_t)k * D + col0 + 4 * c4);
    } else {
      const int c = col0 + 4 * c4 - k;
      rr[i] = f32x4{c == 0 ? 1.f : 0.f, c == -1 ? 1.f : 0.f, c == -2 ? 1.f : 0.f, c == -3 ? 1.f : 0.f};
    }
  }
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int e = tid + i * kThreads, v = e / (D / 8), k8 = (e % (D / 8)) * 8;
    if (e >= XN) break;
    const int64_t vec = vec0 + v < nvec ? vec0 + v : vec0;
    load8<XT>(src, (vec / heads) * src_stride + (vec % heads) * D + k8, xv[i]);
    if (vec0 + v >= nvec) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[i][j] = 0.f;
    }
  }
  if (kind == KIND_K && blockIdx.y == 0 && !p.scan) record_claims(p, vec0, kSV, heads, nvec);
#pragma unroll
  for (int i = 0; i < RI; ++i) {
    const int e = tid + i * kThreads, k = e / (kSC / 4), c4 = e % (kSC / 4);
    if (e < RN) *(f32x4*)&s_r[k][4 * c4] = rr[i];
  }
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int e = tid + i * kThreads, v = e / (D / 8), k8 = (e % (D / 8)) * 8;
    if (e < XN) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s_x[k8 + j][v] = xv[i][j];
    }
  }
  __syncthreads();
  // lane -> vector v (16) x column group cg (4 columns); wave -> key quarter
  const int v = lane >> 2, cg = lane & 3;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  constexpr int KQ = D / 4;
#pragma unroll 8
  for (int kk = 0; kk < KQ; ++kk) {
    const int k = wave * KQ + kk;
    const f32x4 r4 = *(const f32x4*)&s_r[k][4 * cg];
    const double x = s_x[k][v];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = fma(x, (double)r4[j], acc[j]);
  }
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s_red[wave - 1][j][lane] = acc[j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] += s_red[w][j][lane];
  const int64_t vec = vec0 + v;
  if (vec >= nvec) return;
  const float y[4] = {(float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]};
  const int64_t base = vec * D + col0 + 4 * cg;
  if (y_out != nullptr) *(f32x4*)(y_out + base) = f32x4{y[0], y[1], y[2], y[3]};
  if (rot_out != nullptr) store4<XT>(rot_out, base, y);
}

template <int D, int TV, int XT>
__global__ __launch_bounds__(kThreads) void store_rotate_kernel(StoreParams p) {
  const oscar_store_args_v1& a = p.a;
  const int kind = blockIdx.z;
  const int64_t heads = (kind == KIND_Q) ? a.num_q_heads : a.cache.num_kv_heads;
  const int64_t nvec = a.num_tokens * heads;
  const int64_t vec0 = (int64_t)blockIdx.x * TV;
  if (vec0 >= nvec) return;
  const int col0 = blockIdx.y * kCols;
  const int tid = threadIdx.x;

  const void* src = kind == KIND_K ? a.key : (kind == KIND_V ? a.value : a.query);
  const int64_t src_stride = kind == KIND_K ? a.key_stride_token
                           : (kind == KIND_V ? a.value_stride_token : a.query_stride_token);
  const float* R = (kind == KIND_V) ? a.rv : a.rk;
  void* rot_out = kind == KIND_K ? a.key_rot : (kind == KIND_V ? a.value_rot : a.query_rot);
  float* y_out = (kind == KIND_Q) ? nullptr : p.y + (int64_t)kind * a.num_tokens * heads * D;

  // ---- one batch of loads: this block's 64 columns of R and its TV input vectors
  __shared__ __attribute__((aligned(16))) float s_r[D][kCols];
  __shared__ float s_x[D][TV + 1];
  constexpr int RV = D * kCols / 4 / kThreads;       // float4 of R per thread
  constexpr int XV = TV * (D / 8) / kThreads;        // 8-element x loads per thread
  static_assert(RV >= 1 && (TV * (D / 8)) % kThreads == 0, "tile shape");
  f32x4 rr[RV];
  float xv[XV][8];
#pragma unroll
  for (int i = 0; i < RV; ++i) {
    const int e = tid + i * kThreads, k = e / (kCols / 4), c4 = e % (kCols / 4);
    if (R != nullptr) {
      rr[i] = *(const f32x4*)(R + (int64_t)k * D + col0 + 4 * c4);
    } else {
      const int c = col0 + 4 * c4 - k;
      rr[i] = f32x4{c == 0 ? 1.f : 0.f, c == -1 ? 1.f : 0.f, c == -2 ? 1.f : 0.f, c == -3 ? 1.f : 0.f};
    }
  }
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int e = tid + i * kThreads, v = e / (D / 8), k8 = (e % (D / 8)) * 8;
    const int64_t vec = vec0 + v < nvec ? vec0 + v : vec0;
    const int64_t t = vec / heads, h = vec % heads;
    load8<XT>(src, t * src_stride + h * D + k8, xv[i]);
    if (vec0 + v >= nvec) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[i][j] = 0.f;
    }
  }

  if (kind == KIND_K && blockIdx.y == 0 && !p.scan) record_claims(p, vec0, TV, heads, nvec);

#pragma unroll
  for (int i = 0; i < RV; ++i) {
    const int e = tid + i * kThreads, k = e / (kCols / 4), c4 = e % (kCols / 4);
    *(f32x4*)&s_r[k][4 * c4] = rr[i];
  }
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int e = tid + i * kThreads, v = e / (D / 8), k8 = (e % (D / 8)) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) s_x[k8 + j][v] = xv[i][j];
  }
  __syncthreads();

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
#pragma unroll 8
  for (int k = 0; k < D; ++k) {
    const f32x4 r4 = *(const f32x4*)&s_r[k][4 * cg];
    const double r0 = r4[0], r1 = r4[1], r2 = r4[2], r3 = r4[3];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const double x = s_x[k][rg * RPT + i];
      acc[i][0] = fma(x, r0, acc[i][0]);
      acc[i][1] = fma(x, r1, acc[i][1]);
      acc[i][2] = fma(x, r2, acc[i][2]);
      acc[i][3] = fma(x, r3, acc[i][3]);
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t vec = vec0 + rg * RPT + i;
    if (vec >= nvec) continue;
    const float y[4] = {(float)acc[i][0], (float)acc[i][1], (float)acc[i][2], (float)acc[i][3]};
    const int64_t base = vec * D + col0 + cg * 4;
    if (y_out != nullptr) *(f32x4*)(y_out + base) = f32x4{y[0], y[1], y[2], y[3]};
    if (rot_out != nullptr) store4<XT>(rot_out, base, y);
  }
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

// Where one vector (kind K or V of token t) goes: slot, seat, whether this token is
// the last writer of each, and its request's length and query end (for the window
// rule).  Winners of duplicate slots / seats come from the claims (SCAN false) or
// from scanning slot_mapping (SCAN true).  Computed by one wave, wave-uniform.
struct Dest {
  int64_t slot, seat, seq, end;
  bool valid, slot_win, seat_win;
};

template <bool SCAN>
__device__ Dest vector_dest(const StoreParams& p, int kind, int64_t t, int64_t epoch) {
  const oscar_store_args_v1& a = p.a;
  const int lane = threadIdx.x & 63;
  const int64_t bs = a.cache.block_size;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  Dest d{};
  // ---- one round of loads: slot, the request table (and, for a scan call, every
  // slot of the call)
  const int64_t slot = a.slot_mapping[t];
  // request of token t: the last r < num_reqs with min(qsl[r], num_tokens) <= t; its
  // length and query end come from the same loads (qsl is non-decreasing)
  int64_t seq = 0, end = 0;
  if (window) {
    for (int c0 = 0; c0 < a.num_reqs; c0 += 64) {
      const int r = c0 + lane;
      const bool in = r < a.num_reqs;
      const int64_t st = in ? a.query_start_loc[r] : a.num_tokens;
      const int64_t nx = in ? a.query_start_loc[r + 1] : a.num_tokens;
      const int64_t sq = in ? a.seq_lens[r] : 0;
      const int64_t start = st < a.num_tokens ? st : a.num_tokens;
      const uint64_t bal = __ballot(in && start <= t);
      if (bal) {
        const int last = 63 - __builtin_clzll(bal);
        seq = __shfl(sq, last);
        end = __shfl(nx, last);
      }
    }
  }
  d.slot = slot;
  d.seq = seq;
  d.end = end;
  d.valid = slot >= 0 && slot < p.capacity;
  if (!d.valid) return d;
  const int64_t seat = a.stage_mode != OSCAR_STAGE_NONE ? seat_of(slot, bs, a.staging.rows) : 0;
  d.seat = seat;
  bool slot_win, seat_win;
  if constexpr (SCAN) {
    // last writer: no later valid token of the call has the same slot / seat
    bool later_slot = false, later_seat = false;
    for (int64_t c0 = 0; c0 < a.num_tokens; c0 += 64) {
      const int64_t t2 = c0 + lane;
      const int64_t s2 = t2 < a.num_tokens ? a.slot_mapping[t2] : -1;
      const bool later = t2 > t && s2 >= 0 && s2 < p.capacity;
      later_slot |= later && s2 == slot;
      if (window) later_seat |= later && seat_of(s2 < 0 ? 0 : s2, bs, a.staging.rows) == seat;
    }
    slot_win = !__any(later_slot);
    seat_win = !__any(later_seat);
    // standalone KV update: every written seat loses its window copy
    if (a.stage_mode == OSCAR_STAGE_INVALIDATE && kind == KIND_K && lane == 0) a.staging.owner[seat] = -1;
  } else {
    // ---- second round: the claims
    const long long mine = claim_value(epoch, t);
    slot_win = (long long)a.slot_claims[slot] == mine;
    seat_win = window && (long long)a.seat_claims[seat] == mine;
  }
  d.slot_win = slot_win;
  d.seat_win = seat_win;
  return d;
}

// Quantize, pack and scatter one rotated vector (kind K or V of token t, kv head h,
// destination d) held by one wave (lane b < D / 4: elements 4b..4b+3 in x4), with
// the staging window and owner tag of its seat.
template <int D>
__device__ void quant_vector(const StoreParams& p, int kind, int64_t t, int64_t h, const Dest& d, f32x4 x4,
                             float* row, float* clip_slot) {
  constexpr int NL = D / 4;  // lanes holding 4 elements (one packed byte) each
  const oscar_store_args_v1& a = p.a;
  const int64_t hk = a.cache.num_kv_heads;
  const int lane = threadIdx.x & 63;
  const bool active = lane < NL;
  const int64_t bs = a.cache.block_size;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  if (!d.valid) return;
  const int64_t slot = d.slot, seat = d.seat, seq = d.seq, end = d.end;
  const bool slot_win = d.slot_win, seat_win = d.seat_win;
  const int64_t blk = slot / bs, off = slot % bs;
  if (active) *(f32x4*)&row[4 * lane] = x4;

  if (window && seat_win) {
    const int64_t pos = seq - end + t;
    const bool keep = (pos >= seq - a.recent_tokens) || (pos < a.sink_tokens_eff);
    if (kind == KIND_K && lane == 0) a.staging.owner[seat] = keep ? blk : -1;
    if (keep && active) {
      float* dst = (kind == KIND_K ? a.staging.stage_k : a.staging.stage_v) + (seat * hk + h) * D;
      *(f32x4*)&dst[4 * lane] = x4;
    }
  }
  if (!slot_win) return;

  const float clip = kind == KIND_K ? a.k_clip_ratio : a.v_clip_ratio;
  float thr = INFINITY;
  if (clip > 0.f) {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    int idx = (int)(clip * (float)D);
    if (idx > D - 1) idx = D - 1;
    thr = clip_threshold<D>(row, idx, clip_slot);
  }
  // lane b handles byte b = elements 4b..4b+3
  float x[4];
  float vmin = INFINITY, vmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = active ? x4[j] : 0.f;
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

template <int D, bool SCAN>
__global__ __launch_bounds__(kThreads) void store_quant_kernel(StoreParams p) {
  const oscar_store_args_v1& a = p.a;
  const int kind = blockIdx.y;  // K or V
  const int64_t hk = a.cache.num_kv_heads;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // this call's epoch (word1, set by the rotate launch); word0 takes it for the next
  // call (no other quant workgroup reads word0).  Scan calls use no claims.
  int64_t epoch = 0;
  if constexpr (!SCAN) {
    epoch = a.epoch_counter[1];
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) a.epoch_counter[0] = epoch;
  }
  const int64_t vec = (int64_t)blockIdx.x * (kThreads / 64) + wave;
  if (vec >= a.num_tokens * hk) return;
  const float* y = p.y + ((int64_t)kind * a.num_tokens * hk + vec) * D;
  const f32x4 x4 = *(const f32x4*)(y + 4 * (lane < D / 4 ? lane : 0));
  __shared__ float rows[kThreads / 64][D];
  __shared__ float clip_slot[kThreads / 64];
  const Dest d = vector_dest<SCAN>(p, kind, vec / hk, epoch);
  quant_vector<D>(p, kind, vec / hk, vec % hk, d, x4, rows[wave], &clip_slot[wave]);
}

// Calls of at most kFusedTokens tokens (decode and MTP steps): one launch of
// workgroups (token, vectors, column slice).  A workgroup rotates its vectors -- one
// K or V vector (token, kv head), or kQPW query heads of a token -- for one slice of
// kSliceCols output columns, so that no compute unit streams more than D x kSliceCols
// of R: each thread loads RPT rows x 4 columns of the slice straight into registers,
// the products accumulate in fp64 and the KP parts of the contraction are added in
// order (the fp32 result is the correctly rounded one).  Query slices go to
// query_rot.  K / V slices go to the read-path copies and to the workspace; the last
// slice workgroup of a vector to arrive (one counter per vector that atomicInc wraps
// back to zero) reads the whole vector back and quantizes, packs and scatters it in
// place (quant_vector, winners by scanning).  The slices pass through the workspace
// with agent-scope stores and loads, which bypass the per-XCD L2, ordered by the
// store wait, the barrier and the counter; an agent-scope fence would instead write
// back and invalidate the whole L2 in every workgroup.
constexpr int64_t kFusedTokens = 64;
constexpr int kQPW = 2;         // query heads per fused workgroup
constexpr int kSliceCols = 128;  // output columns per fused workgroup
constexpr int kSmallThreads = 512;

template <int D, int XT>
__global__ __launch_bounds__(kSmallThreads) void store_small_kernel(StoreParams p) {
  constexpr int SC = D < kSliceCols ? D : kSliceCols;
  constexpr int NS = D / SC;            // column slices of a vector
  constexpr int CG = SC / 4;            // 4-column groups of a slice
  constexpr int KP = kSmallThreads / CG;     // parts of the contraction
  constexpr int RPT = D / KP;           // rows of R per thread
  static_assert(RPT >= 1 && D % KP == 0 && kQPW * 4 * CG <= kSmallThreads, "slice shape");
  const oscar_store_args_v1& a = p.a;
  const int64_t hk = a.cache.num_kv_heads;
  const int64_t t = blockIdx.x;
  const int yb = blockIdx.y;
  const int c0 = blockIdx.z * SC;
  const int kind = yb < hk ? KIND_K : (yb < 2 * hk ? KIND_V : KIND_Q);
  const int64_t h0 = kind == KIND_K ? yb : (kind == KIND_V ? yb - hk : (int64_t)(yb - 2 * hk) * kQPW);
  const int64_t heads = kind == KIND_Q ? a.num_q_heads : hk;
  const int nv = kind == KIND_Q ? (heads - h0 < kQPW ? (int)(heads - h0) : kQPW) : 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid % CG, kp = tid / CG;
  const void* src = kind == KIND_K ? a.key : (kind == KIND_V ? a.value : a.query);
  const int64_t src_stride = kind == KIND_K ? a.key_stride_token
                           : (kind == KIND_V ? a.value_stride_token : a.query_stride_token);
  const float* R = (kind == KIND_V) ? a.rv : a.rk;
  void* rot_out = kind == KIND_K ? a.key_rot : (kind == KIND_V ? a.value_rot : a.query_rot);

  __shared__ float s_x[kQPW][D];
  __shared__ double s_red[KP][kQPW * 4 * CG];
  __shared__ float s_y[kQPW][SC];
  __shared__ float s_row[D];
  __shared__ float s_clip;
  __shared__ int s_last;
  // this thread's rows kp + KP * i of the slice: issued first, used after the barrier
  f32x4 r4[RPT];
  if (R != nullptr) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) r4[i] = *(const f32x4*)(R + (int64_t)(kp + KP * i) * D + c0 + 4 * cg);
  }
  // the destination of a K / V vector: its loads overlap the rotation (only the last
  // slice to arrive uses it)
  Dest dest{};
  if (kind != KIND_Q && wave == 0) dest = vector_dest<true>(p, kind, t, 0);
  // the input vectors (fp32 in LDS; slots past nv are zero)
  for (int e = tid; e < kQPW * D; e += kSmallThreads)
    if (e >= nv * D) s_x[e / D][e % D] = 0.f;
  for (int e = tid; e < nv * (D / 8); e += kSmallThreads) {
    const int v = e / (D / 8), k8 = (e % (D / 8)) * 8;
    float xv[8];
    load8<XT>(src, t * src_stride + (h0 + v) * D + k8, xv);
#pragma unroll
    for (int j = 0; j < 8; ++j) s_x[v][k8 + j] = xv[j];
  }
  __syncthreads();
  double acc[kQPW][4];
  if (R != nullptr) {
#pragma unroll
    for (int v = 0; v < kQPW; ++v)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[v][j] = 0.0;
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int v = 0; v < kQPW; ++v) {
        const double x = s_x[v][kp + KP * i];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[v][j] = fma(x, (double)r4[i][j], acc[v][j]);
      }
  } else {
#pragma unroll
    for (int v = 0; v < kQPW; ++v)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[v][j] = kp == 0 ? (double)s_x[v][c0 + 4 * cg + j] : 0.0;
  }
  // the KP parts to LDS; thread e < kQPW * SC adds the parts of output e in order
#pragma unroll
  for (int v = 0; v < kQPW; ++v)
#pragma unroll
    for (int j = 0; j < 4; ++j) s_red[kp][(v * 4 + j) * CG + cg] = acc[v][j];
  __syncthreads();
  if (tid < kQPW * 4 * CG) {
    double sum = 0.0;
#pragma unroll 8
    for (int w = 0; w < KP; ++w) sum += s_red[w][tid];
    const int v = tid / (4 * CG), j = (tid / CG) % 4, g4 = tid % CG;
    s_y[v][4 * g4 + j] = (float)sum;
  }
  __syncthreads();
  if (tid < kQPW * CG) {
    const int v = tid / CG, g4 = tid % CG;
    if (v < nv) {
      const f32x4 y4 = *(const f32x4*)&s_y[v][4 * g4];
      float y[4] = {y4[0], y4[1], y4[2], y4[3]};
      const int64_t hq = kind == KIND_Q ? a.num_q_heads : hk;
      if (rot_out != nullptr) store4<XT>(rot_out, (t * hq + h0 + v) * D + c0 + 4 * g4, y);
      if (kind != KIND_Q) {
        // agent-coherent stores (past this XCD's L2), read back the same way below
        float* yw = p.y + (((int64_t)kind * a.num_tokens + t) * hk + h0) * D + c0 + 4 * g4;
#pragma unroll
        for (int j = 0; j < 4; ++j) __hip_atomic_store(yw + j, y[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (kind == KIND_Q) return;
  // the slice is written (stores complete before the barrier): count it in; the last
  // of the vector's slices to arrive goes on
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if constexpr (NS > 1) {
    if (tid == 0)
      s_last = atomicInc(&a.arrivals[((int64_t)kind * a.num_tokens + t) * hk + h0], NS - 1) == NS - 1;
    __syncthreads();
    if (!s_last) return;
  }
  if (wave != 0) return;
  const float* yv = p.y + (((int64_t)kind * a.num_tokens + t) * hk + h0) * D + 4 * (lane < D / 4 ? lane : 0);
  f32x4 x4;
#pragma unroll
  for (int j = 0; j < 4; ++j) x4[j] = __hip_atomic_load(yv + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  quant_vector<D>(p, kind, t, h0, dest, x4, s_row, &s_clip);
}

template <int D, int TV>
void launch_rotate(const StoreParams& p, dim3 grid, hipStream_t s) {
  dim3 block(kThreads);
  if (p.a.kv_dtype == OSCAR_BF16) hipLaunchKernelGGL((store_rotate_kernel<D, TV, OSCAR_BF16>), grid, block, 0, s, p);
  else if (p.a.kv_dtype == OSCAR_F16) hipLaunchKernelGGL((store_rotate_kernel<D, TV, OSCAR_F16>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((store_rotate_kernel<D, TV, OSCAR_F32>), grid, block, 0, s, p);
}

template <int D>
int launch_store(const StoreParams& p, int64_t kv_vec, int64_t q_vec, hipStream_t s) {
  if (p.a.num_tokens <= kFusedTokens && p.scan) {
    const int64_t hk = p.a.cache.num_kv_heads;
    const int64_t qg = q_vec ? (p.a.num_q_heads + kQPW - 1) / kQPW : 0;
    dim3 grid((unsigned)p.a.num_tokens, (unsigned)(2 * hk + qg), (unsigned)(D < kSliceCols ? 1 : D / kSliceCols));
    if (p.a.kv_dtype == OSCAR_BF16) hipLaunchKernelGGL((store_small_kernel<D, OSCAR_BF16>), grid, dim3(kSmallThreads), 0, s, p);
    else if (p.a.kv_dtype == OSCAR_F16) hipLaunchKernelGGL((store_small_kernel<D, OSCAR_F16>), grid, dim3(kSmallThreads), 0, s, p);
    else hipLaunchKernelGGL((store_small_kernel<D, OSCAR_F32>), grid, dim3(kSmallThreads), 0, s, p);
    OSCAR_CHECK_LAUNCH("store_small_kernel");
    return 0;
  }
  const int kinds = q_vec ? 3 : 2;
  const int64_t max_vec = kv_vec > q_vec ? kv_vec : q_vec;
  if (max_vec >= 4096) {
    dim3 grid((unsigned)((max_vec + 63) / 64), D / kCols, kinds);
    launch_rotate<D, 64>(p, grid, s);
  } else {
    dim3 grid((unsigned)((max_vec + kSV - 1) / kSV), D / kSC, kinds);
    dim3 block(kThreads);
    if (p.a.kv_dtype == OSCAR_BF16) hipLaunchKernelGGL((store_rotate_small_kernel<D, OSCAR_BF16>), grid, block, 0, s, p);
    else if (p.a.kv_dtype == OSCAR_F16) hipLaunchKernelGGL((store_rotate_small_kernel<D, OSCAR_F16>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((store_rotate_small_kernel<D, OSCAR_F32>), grid, block, 0, s, p);
  }
  OSCAR_CHECK_LAUNCH("store_rotate_kernel");
  dim3 qgrid((unsigned)((kv_vec + 3) / 4), 2);
  if (p.scan) hipLaunchKernelGGL((store_quant_kernel<D, true>), qgrid, dim3(kThreads), 0, s, p);
  else hipLaunchKernelGGL((store_quant_kernel<D, false>), qgrid, dim3(kThreads), 0, s, p);
  OSCAR_CHECK_LAUNCH("store_quant_kernel");
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
  // inputs are read 8 elements (16 or 32 bytes) at a time, outputs written 4 at a time
  const int esz = a.kv_dtype == OSCAR_F32 ? 4 : 2;
  auto misaligned = [&](const void* ptr, int64_t stride) {
    return ptr != nullptr && ((((uintptr_t)ptr) & 15) || ((stride * esz) & 15));
  };
  if (misaligned(a.key, a.key_stride_token) || misaligned(a.value, a.value_stride_token) ||
      (a.query_rot != nullptr && misaligned(a.query, a.query_stride_token)))
    return fail(-22, "oscar_store_v1: key/value/query rows must be 16-byte aligned");
  if ((a.key_rot && (((uintptr_t)a.key_rot) & 15)) || (a.value_rot && (((uintptr_t)a.value_rot) & 15)) ||
      (a.query_rot && (((uintptr_t)a.query_rot) & 15)))
    return fail(-22, "oscar_store_v1: rotated outputs must be 16-byte aligned");
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
    if (a.stage_mode == OSCAR_STAGE_WRITE &&
        ((((uintptr_t)a.staging.stage_k) & 15) || (((uintptr_t)a.staging.stage_v) & 15)))
      return fail(-22, "oscar_store_v1: staging arena must be 16-byte aligned");
  }
  if (a.query_rot != nullptr &&
      (a.query == nullptr || a.num_q_heads <= 0 || a.query_stride_token < a.num_q_heads * D))
    return fail(-22, "oscar_store_v1: query_rot requires query, num_q_heads and a valid stride");
  const int64_t need = oscar_store_workspace_bytes_v1(a.num_tokens, a.cache.num_kv_heads, D);
  if (a.workspace == nullptr || a.workspace_bytes < need || (((uintptr_t)a.workspace) & 15))
    return fail(-22, "oscar_store_v1: 16-byte aligned workspace of %lld bytes required", (long long)need);
  if (a.num_tokens <= kFusedTokens && (a.arrivals == nullptr || (((uintptr_t)a.arrivals) & 3)))
    return fail(-22, "oscar_store_v1: calls of <= %lld tokens need the arrivals counters", (long long)kFusedTokens);
  StoreParams p{a, (float*)a.workspace, a.cache.num_blocks * a.cache.block_size,
                a.num_tokens <= kScanTokens};
  const int64_t kv_vec = a.num_tokens * a.cache.num_kv_heads;
  const int64_t q_vec = (a.query_rot != nullptr) ? a.num_tokens * a.num_q_heads : 0;
  hipStream_t s = (hipStream_t)stream;
  if (D == 256) return launch_store<256>(p, kv_vec, q_vec, s);
  if (D == 128) return launch_store<128>(p, kv_vec, q_vec, s);
  return launch_store<64>(p, kv_vec, q_vec, s);
}
