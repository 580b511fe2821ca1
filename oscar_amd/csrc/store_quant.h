// Device code of the INT2 quantizer shared by the store launches (store.hip) and the
// decode's merge launch, which finishes deferred small stores (oscar_decode_write_v1):
// the store parameters, destinations (last writers, window rule), the sort clip and
// quant_vector (namespace oscar; inline and template definitions, identical in every
// translation unit that includes it).
#pragma once

#include "common.h"

namespace oscar {

enum Kind { KIND_K = 0, KIND_V = 1, KIND_Q = 2 };

typedef float __attribute__((ext_vector_type(2))) f32x2;

// workgroups of the fused launch per kind at most (bounds the per-workgroup exact counts)
constexpr int kMaxFusedGroups = 1024;

// Division of numerators below 2^31 by a divisor fixed for the call, as a multiply-high
// and a shift (Granlund and Montgomery, "Division by Invariant Integers using
// Multiplication", PLDI 1994, section 4): for 2^(l-1) < d <= 2^l and
// m = floor(2^32 (2^l - d) / d) + 1 (below 2^32), floor(n / d) = (mulhi(m, n) + n) >> l
// for every n < 2^32; the sum is formed in 32 bits, exact for n < 2^31 (mulhi(m, n) < n).
struct FastDiv {
  uint32_t d, m, l;
  static FastDiv of(int64_t divisor) {  // divisors outside [1, 2^31) give a placeholder
    const uint32_t d = divisor >= 1 && divisor < (1ll << 31) ? (uint32_t)divisor : 1u;
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    return {d, (uint32_t)((((1ull << l) - d) << 32) / d + 1), l};
  }
};
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) { return (__umulhi(f.m, n) + n) >> f.l; }
__device__ __forceinline__ uint32_t fmod(uint32_t n, const FastDiv& f) { return n - fdiv(n, f) * f.d; }

struct StoreParams {
  oscar_store_args_v1 a;
  float* y;          // small calls: workspace [2][num_tokens][num_kv_heads][D] fp32 (K then V)
  int64_t capacity;  // num_blocks * block_size
  int32_t* exact;    // large calls: [0] K total, [1] V total (written by the exact pass),
                     // [2 + kind * kMaxFusedGroups + w] vectors workgroup w of the fused launch
                     // left to the exact pass, then the lists [kind][nvec] (nvec = num_tokens *
                     // num_kv_heads): workgroup w's entries start at its first vector
  int32_t* flags;    // large calls: [num_tokens] bit 0 = position inside the window
  u32x4* planes;     // large calls: R_k, R_v as fp16 MFMA B fragments [2][D/32][D/16][2][64]
  int32_t* bexp;     // large calls: [2][D] power-of-two column scale of the planes
  float* colnorm;    // large calls: [2][D] ||R_:d||
  int32_t fused_kv_groups;  // large calls: fused workgroups per kind for K and for V
  int32_t deferred;  // small calls of oscar_decode_write_v1: store_small_kernel rotates only
                     // (read-path copies, rotated K / V in y, pending tags); the merge launch
                     // of the decode quantizes (quant_deferred)
  int32_t slots31;   // capacity < 2^31: slots split into block and offset by div_bs
  FastDiv div_hk, div_hq, div_bs, div_rows;  // num_kv_heads, num_q_heads, block_size, staging rows
};

// Owner tag of a seat that a deferred small call rewrites, from its rotation launch to
// its quantization: it matches no block, so a reader in between (the decode of
// oscar_decode_write_v1) treats the seat as the call leaves it -- rewritten or
// invalidated, the old token's FP32 copy is gone either way.
constexpr int64_t kPendingTag = -2;

__device__ __forceinline__ int32_t* exact_counts(const StoreParams& p, int kind) {
  return p.exact + 2 + kind * kMaxFusedGroups;
}
__device__ __forceinline__ int32_t* exact_list(const StoreParams& p, int kind, int64_t nvec) {
  return p.exact + 2 + 2 * kMaxFusedGroups + kind * nvec;
}

__device__ __forceinline__ long long claim_value(int64_t epoch, int64_t token) {
  // 39-bit epoch above a 24-bit token index: 5e11 calls before the counter saturates
  return (long long)((epoch << 24) | (token & 0xffffffll));
}
constexpr int64_t kMaxEpoch = (1ll << 39) - 1;

__device__ __forceinline__ int64_t seat_of(int64_t slot, int64_t bs, int64_t rows) {
  return ((slot / bs) % rows) * bs + slot % bs;
}
// the same for a slot in [0, capacity), by the call's fixed divisors where they apply
__device__ __forceinline__ int64_t seat_of(const StoreParams& p, int64_t slot) {
  if (p.slots31) {
    const uint32_t s = (uint32_t)slot, blk = fdiv(s, p.div_bs);
    return (int64_t)fmod(blk, p.div_rows) * p.div_bs.d + (s - blk * p.div_bs.d);
  }
  return seat_of(slot, p.a.cache.block_size, p.a.staging.rows);
}
__device__ __forceinline__ int64_t block_of(const StoreParams& p, int64_t slot) {
  return p.slots31 ? (int64_t)fdiv((uint32_t)slot, p.div_bs) : slot / p.a.cache.block_size;
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

// Sort-clip threshold (backend.py:140-145): the idx-th smallest |x| (0-based) of a
// D-vector held by one wave, lane l < D / 4 holding elements 4l .. 4l + 3 in x4.
// Selected on the magnitude bits (the order of |x|; NaN above inf, as a sort puts it
// last): the answer a is the largest v with count(|x| < v) <= idx, the (D - idx)-th
// largest element, found by bisection of [lo, hi) with a in [lo, hi), each count four
// ballots of the wave.  hi = the maximum + 1; lo = the minimum over the D / 16 lane
// quads of each quad's k-th largest, k = 1 while D - idx <= D / 16, 2 while <= D / 8
// (every quad holds k elements >= lo, so at least D - idx do and a >= lo), else 0.
// Once the interval holds exactly one element (c_hi - c_lo == 1) that element is the
// answer, gathered by an OR over the wave; an interval one value wide gives lo (ties).
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  return __float_as_uint(wave_reduce(__uint_as_float(x), [](float a, float b) {
    return __uint_as_float(min(__float_as_uint(a), __float_as_uint(b)));
  }));
}
template <int D>
__device__ float wave_kth_abs(f32x4 x4, int idx) {
  const bool active = (int)(threadIdx.x & 63) < D / 4;
  uint32_t u[4];
  uint32_t m1 = 0, m2 = 0;  // this lane's largest and second largest
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u[j] = active ? (__float_as_uint(x4[j]) & 0x7fffffffu) : 0xffffffffu;
    const uint32_t w = active ? u[j] : 0u;
    m2 = max(m2, min(m1, w));
    m1 = max(m1, w);
  }
  auto quad_top2 = [&](uint32_t o1, uint32_t o2) {  // merge another lane's two largest
    m2 = max(min(m1, o1), max(m2, o2));
    m1 = max(m1, o1);
  };
  quad_top2(__float_as_uint(dpp_row<kDppXor1>(__uint_as_float(m1))), __float_as_uint(dpp_row<kDppXor1>(__uint_as_float(m2))));
  quad_top2(__float_as_uint(dpp_row<kDppXor2>(__uint_as_float(m1))), __float_as_uint(dpp_row<kDppXor2>(__uint_as_float(m2))));
  const int need = D - idx;
  uint32_t lo = wave_min_u32(active ? (need <= D / 16 ? m1 : (need <= D / 8 ? m2 : 0u)) : 0xffffffffu);
  uint32_t hi = ~wave_min_u32(~m1) + 1u;  // the maximum + 1 (<= 2^31)
  int c_lo = 0, c_hi = D;  // c_lo: a lower bound of count(|x| < lo) until lo first moves
  while (hi - lo > 1 && c_hi - c_lo > 1) {  // wave-uniform: one vector per wave
    const uint32_t mid = lo + ((hi - lo) >> 1);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) cnt += __popcll(__ballot(u[j] < mid));
    if (cnt <= idx) {
      lo = mid;
      c_lo = cnt;
    } else {
      hi = mid;
      c_hi = cnt;
    }
  }
  // the one element in [lo, hi), its bits kept exactly (NaN payloads included)
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (u[j] >= lo && u[j] < hi) m |= u[j];
  m = __float_as_uint(wave_reduce(__uint_as_float(m), [](float a, float b) {
    return __uint_as_float(__float_as_uint(a) | __float_as_uint(b));
  }));
  return __uint_as_float(c_hi - c_lo == 1 ? m : lo);
}

// Where one vector (kind K or V of token t) goes: slot, seat, whether this token is
// the last writer of each, and whether its position lies inside its request's sink /
// recent window (backend.py:536-541: keep the FP32 copy, else drop the seat).
struct Dest {
  int64_t slot, seat;
  int64_t koff, voff;  // fused kernel: byte offsets of the K and V slots in the caches
  bool valid, slot_win, seat_win, keep;
};

// the window rule for token t of a request of length seq whose queries end at end
__device__ __forceinline__ bool in_window(const oscar_store_args_v1& a, int64_t t, int64_t seq, int64_t end) {
  const int64_t pos = seq - end + t;
  return (pos >= seq - a.recent_tokens) || (pos < a.sink_tokens_eff);
}

// Destination of a small call's vector: winners of duplicate slots / seats by
// scanning slot_mapping.  Computed by one wave, wave-uniform, in two steps so that
// the loads go out early and their results are used late: dest_loads issues every
// load (the token's slot, lane l's request-table entry and lane l's slot of the
// call), dest_finish decides.  A call has at most kFusedTokens (64) tokens, so one
// slot per lane covers it; requests past the first 64 are read in dest_finish.
// The raw reads, all issued at once and without a branch (lanes with nothing to read
// read entry 0 of a valid array); dest_finish masks them.  A select or widening right
// after a read would make the compiler wait for each read in turn.
struct DestLoads {
  int64_t slot;        // slot_mapping[t]
  int64_t s2;          // slot_mapping[lane] (lanes past the call: entry 0)
  int32_t st, nx, sq;  // query_start_loc[lane], [lane + 1], seq_lens[lane] (lanes past the
                       // requests, or no window: entries 0 and 1 of slot_mapping's words)
};

__device__ __forceinline__ DestLoads dest_loads(const StoreParams& p, int64_t t) {
  const oscar_store_args_v1& a = p.a;
  const int lane = threadIdx.x & 63;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  const int32_t* qsl = window ? a.query_start_loc : reinterpret_cast<const int32_t*>(a.slot_mapping);
  const int32_t* sql = window ? a.seq_lens : reinterpret_cast<const int32_t*>(a.slot_mapping);
  const int r = window && lane < a.num_reqs ? lane : 0;
  DestLoads l;
  l.slot = a.slot_mapping[t];
  l.s2 = a.slot_mapping[lane < a.num_tokens ? lane : 0];
  l.st = qsl[r];
  l.nx = qsl[r + 1];
  l.sq = sql[r];
  return l;
}

__device__ inline Dest dest_finish(const StoreParams& p, int kind, int64_t t, const DestLoads& l) {
  const oscar_store_args_v1& a = p.a;
  const int lane = threadIdx.x & 63;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  Dest d{};
  const int64_t slot = l.slot;
  // request of token t: the last r < num_reqs with min(qsl[r], num_tokens) <= t; its
  // length and query end come from the same loads (qsl is non-decreasing)
  int64_t seq = 0, end = 0;
  if (window) {
    for (int c0 = 0; c0 < a.num_reqs; c0 += 64) {
      const int r = c0 + lane;
      const bool in = r < a.num_reqs;
      int64_t st = in ? l.st : a.num_tokens, nx = in ? l.nx : a.num_tokens, sq = in ? l.sq : 0;
      if (c0 > 0) {
        st = in ? a.query_start_loc[r] : a.num_tokens;
        nx = in ? a.query_start_loc[r + 1] : a.num_tokens;
        sq = in ? a.seq_lens[r] : 0;
      }
      const int64_t start = st < a.num_tokens ? st : a.num_tokens;
      // the shuffles run whatever the ballot (so the reads stay where dest_loads issued
      // them instead of sinking into the taken branch)
      const uint64_t bal = __ballot(in && start <= t);
      const int last = bal ? 63 - __builtin_clzll(bal) : 0;
      const int64_t sq_last = __shfl(sq, last), nx_last = __shfl(nx, last);
      if (bal) {
        seq = sq_last;
        end = nx_last;
      }
    }
  }
  d.slot = slot;
  d.keep = window && in_window(a, t, seq, end);
  d.valid = slot >= 0 && slot < p.capacity;
  if (!d.valid) return d;
  const int64_t seat = a.stage_mode != OSCAR_STAGE_NONE ? seat_of(p, slot) : 0;
  d.seat = seat;
  // last writer: no later valid token of the call has the same slot / seat
  {
    const int64_t t2 = lane, s2 = lane < a.num_tokens ? l.s2 : -1;
    const bool later = t2 > t && s2 >= 0 && s2 < p.capacity;
    const bool later_slot = later && s2 == slot;
    const bool later_seat = window && later && seat_of(p, s2) == seat;
    d.slot_win = !__any(later_slot);
    d.seat_win = window && !__any(later_seat);
    // standalone KV update: every written seat loses its window copy
    if (a.stage_mode == OSCAR_STAGE_INVALIDATE && kind == KIND_K && lane == 0) a.staging.owner[seat] = -1;
  }
  return d;
}

// Quantize, pack and scatter one rotated vector (kind K or V of token t, kv head h,
// destination d) held by one wave (lane b < D / 4: elements 4b..4b+3 in x4), with
// the staging window and owner tag of its seat.
template <int D>
__device__ void quant_vector(const StoreParams& p, int kind, int64_t t, int64_t h, const Dest& d, f32x4 x4) {
  constexpr int NL = D / 4;  // lanes holding 4 elements (one packed byte) each
  const oscar_store_args_v1& a = p.a;
  const int64_t hk = a.cache.num_kv_heads;
  const int lane = threadIdx.x & 63;
  const bool active = lane < NL;
  const int64_t bs = a.cache.block_size;
  const bool window = a.stage_mode == OSCAR_STAGE_WRITE;
  if (!d.valid) return;
  const int64_t slot = d.slot, seat = d.seat;
  const bool slot_win = d.slot_win, seat_win = d.seat_win;
  const int64_t blk = block_of(p, slot), off = slot - blk * bs;

  if (window && seat_win) {
    const bool keep = d.keep;
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
    int idx = (int)(clip * (float)D);
    if (idx > D - 1) idx = D - 1;
    thr = wave_kth_abs<D>(x4, idx);
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

// Store launch shared by oscar_store_v1 and oscar_decode_write_v1 (store.hip): checks
// the arguments (messages prefixed by fn), then launches the store on stream; with
// defer and a call of at most 64 tokens only the rotation (store_small_kernel with
// p.deferred = 1: read-path copies, rotated K / V in p.y, pending tags), the
// quantization being left to quant_deferred in the decode's merge launch.  *out
// receives the parameters; returns 0, or the negative error.
int store_launch(const oscar_store_args_v1* args, void* stream, bool defer, const char* fn, StoreParams* out);

}  // namespace oscar
