// Streaming split-K paged attention over the packed INT2 history (gfx950).
//
// Replaces oscar_ascend/kernels/slab_attention.py:376-476 (slab_attention) for
// requests whose rows (query tokens x heads per KV head) fit one 32-row MFMA tile:
// decode, MTP verification (1 + 3 drafts x 6 heads = 24 rows) and cache-only decode.
// Semantics follow streaming_attention.py:134-196: query i of a request with n_q
// queries and length seq sees keys [0, seq - n_q + i + 1); history keys come from
// the packed cache unless the staging owner tag of their seat equals the physical
// block (then the FP32 staged value is used); keys >= the history length come from
// the current (rotated, unquantized) chunk.
//
// Work decomposition: the host plan (oscar_attn_plan_v1) cuts every (request,
// kv-head) key range into items of whole 32-token tiles, interleaved so that all
// items of a group land on the same XCD.  One 256-thread workgroup (4 waves, one
// per SIMD) per item; wave w takes tiles w, w+4, ...  Pages hold a multiple of 32
// tokens, so a tile never straddles a page: its block id, seat row and in-page
// offset are wave-uniform scalars.  The four wave partials are merged in LDS and
// the item partial (normalised O in MFMA register order, natural-log LSE) goes to
// the workspace with coalesced 16-byte stores; attn_merge_kernel combines the items
// of each group (FP32 LSE merge, slab_attention.py:341-356) into out_rot / lse.
//
// Memory pipeline: each wave keeps kDepth tiles of packed data in flight (codes,
// scales/zeros and owner tags of its next tiles are loaded into registers while the
// current tile is computed), so HBM latency is paid once per wave, not per tile.
//
// Tile math (one wave, 32 tokens x 32 rows, S^T = K Q^T then O^T += V^T P^T):
//  * QK (bf16 MFMA 32x32x16): the K operand holds exactly the reference's history
//    values bf16(fp16(code*scale + zero)).  A token has only four of them; they form
//    an 8-byte table and one v_perm_b32 per bf16 pair looks the codes up (selector
//    2*code, 2*code+1), so scores and LSE carry the reference rounding.
//  * PV fast tiles (INT2 history, no staged token, no mask; fp16 MFMA): V codes go
//    to LDS in their natural layout and come back transposed with ds_read_b64_tr_b8
//    (8 tokens x 1 byte = 4 codes per lane); one v_perm and one AND per fp16 pair
//    give the subnormal c*2^(2k-24) for code bits 2k..2k+1, the B operand is
//    P' = p*s_V (fp16, round to nearest) and sum_t p*z_V accumulates on the VALU.
//  * slow tiles (staged tokens, current chunk, causal boundary, ragged end, or a
//    score max far above the wave's reference max) are deferred until the fast
//    tiles are done and the accumulators are in value units.  Their K/V values
//    (rounded as the reference does) are built from the codes, the FP32 staged rows
//    (loaded in batched rounds) and the current chunk (copied to LDS once per
//    workgroup); V goes through LDS and is read transposed with ds_read_b64_tr_b16;
//    P is split into bf16 hi + lo parts.
#include <vector>

#include "common.h"

namespace oscar {

namespace {

constexpr int kWaves = 8;            // two waves per SIMD
constexpr int kThreads = kWaves * 64;
constexpr int kSlowWaves = 4;        // waves that run the queued slow tiles
constexpr int kTile = 32;
constexpr int kMaxCur = 32;          // current-chunk tokens of a request (rows <= 32)
constexpr int kMaxItemTokens = 8192; // keys per item (64 tiles per wave)
constexpr int kMaxPages = kMaxItemTokens / kTile + 2;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazy = 8.f;         // max drift (log2 units) before O is rescaled
typedef short __attribute__((ext_vector_type(4))) i16x4;
typedef _Float16 __attribute__((ext_vector_type(2))) f16x2;
typedef __bf16 __attribute__((ext_vector_type(2))) bf16x2;
typedef float __attribute__((ext_vector_type(2))) f32x2;

template <int D>
struct Cfg {
  static constexpr int KSTEPS = D / 16;  // QK contraction steps
  static constexpr int NQ = D / 128;     // 16-byte code vectors per lane half (D/8 bytes)
  static constexpr int NCH = D / 32;     // 16-element chunks per lane half
  static constexpr int NB = D / 4;       // code bytes per token
  static constexpr int MBLK = D / 32;    // PV output blocks (32 d each)
  static constexpr int VROW = D + 8;     // bf16 per row of the slow-tile V buffer
  static constexpr int CPR = 1;          // chunks per staged-row load round
  static constexpr int NV = MBLK * 4 * 64;  // f32x4 of one item partial (register order)
};

struct AttnParams {
  oscar_attn_args_v1 a;
  oscar_staging_v1 st;
  int has_stage;
  int group;     // Hq / Hk
  float* part_o;   // [num_items][32 * D] in MFMA register order
  float* part_lse; // [num_items][32]
};

__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

// exchange with lane l^32
__device__ __forceinline__ float swap_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  // r[0]: lanes 0-31 keep their value, lanes 32-63 receive lanes 0-31's;
  // r[1]: lanes 0-31 receive lanes 32-63's, lanes 32-63 keep theirs.
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// reference history rounding, fp16 then bf16 (streaming_attention.py:124), of a
// pair (a -> low half, b -> high half) with the packed RNE conversions
// v_cvt_pk_f16_f32 / v_cvt_f32_f16 / v_cvt_pk_bf16_f32
__device__ __forceinline__ unsigned hist_pair(float a, float b) {
  const f16x2 h = __builtin_convertvector(f32x2{a, b}, f16x2);
  const f32x2 w = __builtin_convertvector(h, f32x2);
  return __builtin_bit_cast(unsigned, __builtin_convertvector(w, bf16x2));
}
// bf16 pair (RNE) of two floats
__device__ __forceinline__ unsigned bf16_pair(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// PV output block mb, MFMA row m -> d, and the code position of the block
template <int D>
__device__ __forceinline__ int pv_d(int mb, int m) {
  return (D == 256) ? 128 * (mb >> 2) + 4 * m + (mb & 3) : 4 * m + mb;
}
__device__ __forceinline__ int pv_pos(int mb) { return 2 * (mb & 3); }
// slow-tile V buffer column of d-chunk c, element q + 4u (u = 0..3 consecutive)
template <int D>
__device__ __forceinline__ int vbuf_col(int g, int q, int c) {
  return ((D == 256) ? 128 * g + 32 * q : 32 * q + 16 * g) + 4 * c;
}

// token (0..31) of MFMA K-element e for lane half g in PV K-step s
__device__ __forceinline__ int pv_tok(int s, int g, int e) {
  return 16 * s + 4 * g + (e & 3) + 8 * (e >> 2);
}
// token of S^T output register r for lane half g (also the O^T row of register r)
__device__ __forceinline__ int out_tok(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// bf16 pairs (element k, element k+8), k = 0..7, of 16 elements held as two
// 8-element vectors
__device__ __forceinline__ void interleave8(const u32x4& lo, const u32x4& hi, unsigned o[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    o[2 * w] = __builtin_amdgcn_perm(hi[w], lo[w], 0x05040100u);
    o[2 * w + 1] = __builtin_amdgcn_perm(hi[w], lo[w], 0x07060302u);
  }
}

// history value table of one token, bf16(fp16(c*scale + zero)) for c = 0..3
__device__ __forceinline__ void value_table(unsigned scale_zero, unsigned& lo, unsigned& hi) {
  const float s = f16_bits_to_f32(scale_zero & 0xffff), z = f16_bits_to_f32(scale_zero >> 16);
  float v[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(__fmul_rn((float)c, s), z);  // mul, then add
  lo = hist_pair(v[0], v[1]);
  hi = hist_pair(v[2], v[3]);
}

// bf16 pairs (element k, element k+8) of the 16 codes of one code dword
__device__ __forceinline__ void table_pairs(unsigned w, unsigned lo, unsigned hi, unsigned o[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const unsigned y = (w >> (2 * k)) & 0x00030003u;
    o[k] = __builtin_amdgcn_perm(hi, lo, y * 0x202u + 0x01000100u);
  }
}

// bf16 pairs of 16 elements (lo = e0..e7, hi = e8..e15) in the K-step order of lut16:
// (e0,e4) (e1,e5) (e2,e6) (e3,e7) | (e8,e12) (e9,e13) (e10,e14) (e11,e15)
__device__ __forceinline__ void kpairs16(const u32x4& lo, const u32x4& hi, unsigned o[8]) {
  o[0] = __builtin_amdgcn_perm(lo[2], lo[0], 0x05040100u);
  o[1] = __builtin_amdgcn_perm(lo[2], lo[0], 0x07060302u);
  o[2] = __builtin_amdgcn_perm(lo[3], lo[1], 0x05040100u);
  o[3] = __builtin_amdgcn_perm(lo[3], lo[1], 0x07060302u);
  o[4] = __builtin_amdgcn_perm(hi[2], hi[0], 0x05040100u);
  o[5] = __builtin_amdgcn_perm(hi[2], hi[0], 0x07060302u);
  o[6] = __builtin_amdgcn_perm(hi[3], hi[1], 0x05040100u);
  o[7] = __builtin_amdgcn_perm(hi[3], hi[1], 0x07060302u);
}

// the four history values of a token as byte tables: t_lo = low bytes of the bf16
// values for codes 0..3, t_hi = their high bytes
__device__ __forceinline__ void byte_tables(unsigned scale_zero, unsigned& t_lo, unsigned& t_hi) {
  unsigned lo, hi;
  value_table(scale_zero, lo, hi);
  t_lo = __builtin_amdgcn_perm(hi, lo, 0x06040200u);
  t_hi = __builtin_amdgcn_perm(hi, lo, 0x07050301u);
}

// bf16 values of the 16 codes of one code dword (byte j holds elements 4j..4j+3 at
// bits 2k), in the pair order of kpairs16.  Per k: the four codes 4j + k as bytes
// select table bytes directly (v_perm_b32 selectors 0..3), one perm each for the low
// and high bytes, then two perms interleave them into bf16 pairs: 23 VALU per dword.
__device__ __forceinline__ void lut16(unsigned w, unsigned t_lo, unsigned t_hi, unsigned o[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const unsigned x = (w >> (2 * k)) & 0x03030303u;
    const unsigned lo = __builtin_amdgcn_perm(t_hi, t_lo, x);
    const unsigned hi = __builtin_amdgcn_perm(t_lo, t_hi, x);
    o[k] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);      // (e_k, e_4+k)
    o[4 + k] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // (e_8+k, e_12+k)
  }
}

template <int D>
struct TileRegs {
  u32x4 k[Cfg<D>::NQ];  // this lane's half of the K codes
  u32x4 v[Cfg<D>::NQ];  // this lane's half of the V codes
  u32x2 meta;           // K scale, K zero, V scale, V zero (fp16)
  int64_t own;          // owner tag of the token's staging seat
  int blk;              // physical block of the tile (0 off the history)
};

template <int D>
__global__ __launch_bounds__(kThreads, 1) void attn_main_kernel(AttnParams P) {
  using C = Cfg<D>;
  const oscar_attn_args_v1& A = P.a;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = lane & 31, g = lane >> 5;
  // item record: request, kv head | query count << 16, tiles first + stride * j for
  // j < count (32 keys each), partial slot, the request's first query token and length
  const int32_t* it = A.items + (int64_t)blockIdx.x * OSCAR_WORK_INTS;
  const int req = it[0], kvh = it[1] & 0xffff, nq = it[1] >> 16;
  const int first = it[2], stride = it[3], count = it[4], part = it[5];
  const int qa = it[6], seq = it[7];
  const int G = P.group;
  const bool has_new = A.k_new != nullptr;
  const int hist = has_new ? seq - nq : seq;
  const int nrows = nq * G;
  const int bs = (int)A.cache.block_size;  // a multiple of 32
  const int64_t hk = A.cache.num_kv_heads;
  if (part < 0 || part >= A.num_items) return;
  // an item that breaks oscar_attn_plan_v1's rules poisons its partial (NaN LSE, so
  // the merged rows are NaN) instead of reading out of bounds
  if (req < 0 || req >= A.num_reqs || kvh >= hk || nq < 1 || nrows > 32 || hist < 0 ||
      qa < 0 || qa + nq > A.num_tokens || first < 0 || stride < 1 || count < 0 ||
      count > kMaxItemTokens / kTile ||
      (count > 0 && (first + (int64_t)stride * (count - 1)) * kTile >= seq)) {
    if (tid < 32) P.part_lse[(int64_t)part * 32 + tid] = NAN;
    return;
  }
  const int lim0 = seq - nq + 1;                              // first key masked for a row
  const int fast_end = hist < lim0 ? hist : lim0;             // fast tiles end at or before
  auto tile_t0 = [&](int j) { return (first + stride * j) * kTile; };  // first key of item tile j

  // LDS
  __shared__ int32_t s_blk[kMaxPages];                 // block ids of the item's pages
  __shared__ int32_t s_seat[kMaxPages];                // their seat-row base (blk % rows) * bs
  __shared__ __attribute__((aligned(16))) uint8_t s_vcode[kWaves][kTile * C::NB];
  __shared__ __attribute__((aligned(16))) float s_cst[kWaves][2][kTile];
  __shared__ __attribute__((aligned(16))) float s_ml[kWaves][2][32];
  __shared__ __attribute__((aligned(16))) uint16_t s_cur[2][kMaxCur][D];  // current K / V
  __shared__ __attribute__((aligned(16))) u32x4 s_q[C::KSTEPS][64];        // Q^T operand
  __shared__ int32_t s_nslow[kWaves];
  __shared__ int16_t s_slow[kMaxItemTokens / kTile];   // queued slow tiles of all waves
  // union: slow-tile V values (bf16, permuted columns) / cross-wave merge rounds
  constexpr int kMergeBytes = kWaves * 2 * 4 * 64 * 16, kSlowBytes = kSlowWaves * kTile * C::VROW * 2;
  __shared__ __attribute__((aligned(16))) uint8_t s_big[kMergeBytes > kSlowBytes ? kMergeBytes : kSlowBytes];
  const unsigned st_rows = (unsigned)P.st.rows;

  // wave w takes item tiles j = w + kWaves * i, i < my (my <= 32)
  const int my = count > wave ? (count - 1 - wave) / kWaves + 1 : 0;
  const uint8_t* kbase = A.cache.k + (int64_t)kvh * A.cache.k_stride[2];
  const uint8_t* vbase = A.cache.v + (int64_t)kvh * A.cache.v_stride[2];
  const int64_t ks0 = A.cache.k_stride[0], ks1 = A.cache.k_stride[1];
  const int64_t vs0 = A.cache.v_stride[0], vs1 = A.cache.v_stride[1];
  const int64_t* owner = P.st.owner;

  // ---- prologue.  Lane i < my of each wave fetches the page of the wave's tile i
  // (kept in a register for the fast pass, and in LDS for the slow pass, which may
  // run the tile on another wave), so the first tile loads go out before the
  // workgroup barrier that publishes the queries and the current chunk.
  int wblk = 0, wseat = 0;
  if (lane < my) {
    const int j = wave + kWaves * lane;
    const int t0 = tile_t0(j);
    if (t0 < hist) {
      const int32_t b = A.block_table[(int64_t)req * A.block_table_stride + t0 / bs];
      // ids outside the cache are clamped (the host validates tables; this keeps a
      // bad table from faulting)
      wblk = (b < 0 || b >= A.cache.num_blocks) ? 0 : b;
    }
    wseat = P.has_stage ? (int)((unsigned)wblk % st_rows) * bs : 0;
    s_blk[j] = wblk;
    s_seat[j] = wseat;
  }

  // page of item tile j < count, first key t0 (wave-uniform): block, in-page offset
  // of t0 and seat-row base; tiles past the history and the clamped placeholder a
  // wave without tiles loads read block 0 at offsets 0..31 (< block_size).  The
  // wave's own tile i comes from lane i of wblk / wseat; other tiles (slow pass,
  // after a barrier) from LDS.
  auto tile_page = [&](int j, int t0, int& blk, int& off0, int& seat0) {
    blk = 0;
    off0 = 0;
    seat0 = 0;
    if (j < count && t0 < hist) {
      off0 = t0 % bs;
      blk = __builtin_amdgcn_readfirstlane(s_blk[j]);
      seat0 = __builtin_amdgcn_readfirstlane(s_seat[j]);
    }
  };

  auto load_tile = [&](int ti, TileRegs<D>& r) {
    const int j = wave + kWaves * ti;
    const int t0 = tile_t0(j);
    const bool real = j < count && t0 < hist;
    const int off0 = real ? t0 % bs : 0;
    r.blk = real ? __builtin_amdgcn_readlane(wblk, ti) : 0;
    const int seat0 = real ? __builtin_amdgcn_readlane(wseat, ti) : 0;
    const int off = off0 + m;
    const uint8_t* ks = kbase + (int64_t)r.blk * ks0 + (int64_t)off * ks1;
    const uint8_t* vs = vbase + (int64_t)r.blk * vs0 + (int64_t)off * vs1;
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) {
      r.k[i] = *(const u32x4*)(ks + 32 + g * (D / 8) + 16 * i);
      r.v[i] = *(const u32x4*)(vs + g * (D / 8) + 16 * i);
    }
    r.meta = *(const u32x2*)ks;
    // without a staging arena the tag is read from the item record (never matches)
    const int64_t* op = P.has_stage ? owner + seat0 + off : (const int64_t*)it;
    r.own = *op;
  };

  // the wave's first two tiles (register slots A and B, see the main loop)
  const int last = my > 0 ? my - 1 : 0;
  TileRegs<D> RA, RB;
  load_tile(0, RA);
  load_tile(1 < last ? 1 : last, RB);

  // current chunk (tail items) and queries to LDS
  bool any_cur_tile = false;
  if (count > 0) any_cur_tile = has_new && tile_t0(count - 1) + kTile > hist;  // tiles ascend
  if (any_cur_tile) {
    constexpr int V8 = D / 8;
    for (int e = tid; e < nq * V8; e += kThreads) {
      const int t = e / V8, col = (e % V8) * 8;
      const int64_t src = (int64_t)(qa + t) * A.kv_new_stride_token + (int64_t)kvh * D + col;
      *(u32x4*)&s_cur[0][t][col] = *(const u32x4*)((const uint16_t*)A.k_new + src);
      *(u32x4*)&s_cur[1][t][col] = *(const u32x4*)((const uint16_t*)A.v_new + src);
    }
  }
  // queries: lane (row n = m, half g) holds q[n][g*D/2 .. +D/2) in the K-step order
  // of the code lookup (kpairs16); the Q^T operand of K-step j for lane l lives at
  // s_q[j][l] (shared by the waves)
  const int n = m;
  const bool row_ok = n < nrows;
  if (wave == 0) {
    const int qtok = qa + (row_ok ? n / G : 0);
    const int qhead = kvh * G + (row_ok ? n % G : 0);
    const uint16_t* qrow = (const uint16_t*)A.q + (int64_t)qtok * A.q_stride_token + (int64_t)qhead * D + g * (D / 2);
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
      u32x4 lo = *(const u32x4*)(qrow + 16 * c);
      u32x4 hi = *(const u32x4*)(qrow + 16 * c + 8);
      if (!row_ok) lo = hi = u32x4{0u, 0u, 0u, 0u};
      unsigned o[8];
      kpairs16(lo, hi, o);
      s_q[2 * c][lane] = u32x4{o[0], o[1], o[2], o[3]};
      s_q[2 * c + 1][lane] = u32x4{o[4], o[5], o[6], o[7]};
    }
  }
  const float c_score = A.scale * kLog2e;  // scores in log2 units
  __syncthreads();
  // Q^T operands are read from LDS at each use (volatile: kept out of registers)
  auto qop = [&](int j) {
    return __builtin_bit_cast(bf16x8, *(const volatile u32x4*)&s_q[j][lane]);
  };

  // ---- running state (per lane row n): reference max m_run (log2 units), sum l, z
  float m_run = -INFINITY, l_run = 0.f, z_run = 0.f;
  f32x16 O[C::MBLK];
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = 0.f;

  // Lazy: the reference max of a row only moves when a tile's max exceeds it by
  // more than kLazy (log2 units), so probabilities stay <= 2^kLazy and the O
  // accumulators (kept in AGPRs by the MFMAs) are touched by the VALU only then.
  auto update_max = [&](float mx) {
    const bool move = mx > m_run + kLazy;  // also true for the first finite max
    if (__any(move)) {
      const float m_new = move ? mx : m_run;
      const float f = (!move || m_run == -INFINITY) ? (move ? 0.f : 1.f) : exp2f(m_run - m_new);
      if (__any(move && m_run != -INFINITY)) {
#pragma unroll
        for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) O[b][r] *= f;
      }
      l_run *= f;
      z_run *= f;
      m_run = m_new;
    }
  };

  // ---------------------------------------------------------------- fast tiles
  // Phase 1 (QK) of tile ti: decides whether the tile is fast (INT2 history only,
  // no staged token, no mask); if so, its V codes and V constants go to this wave's
  // LDS slots and S^T = K Q^T runs with the exact history values looked up per code.
  auto qk_tile = [&](int ti, const TileRegs<D>& r, f32x16& S) -> bool {
    const int t0 = tile_t0(wave + kWaves * ti);
    const int p = t0 + m;
    const bool staged = P.has_stage && p < hist && r.own == (int64_t)r.blk;
    if (!((t0 + kTile <= fast_end) && !__any(staged))) return false;
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) *(u32x4*)&s_vcode[wave][m * C::NB + g * (D / 8) + 16 * i] = r.v[i];
    s_cst[wave][0][m] = f16_bits_to_f32(r.meta[1] & 0xffff);  // both halves write the same
    s_cst[wave][1][m] = f16_bits_to_f32(r.meta[1] >> 16);
    unsigned t_lo, t_hi;
    byte_tables(r.meta[0], t_lo, t_hi);
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) S[r2] = 0.f;
#pragma unroll
    for (int i = 0; i < C::NCH; ++i) {
      unsigned o[8];
      lut16(r.k[i >> 2][i & 3], t_lo, t_hi, o);
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]}),
                                                  qop(2 * i), S, 0, 0, 0);
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{o[4], o[5], o[6], o[7]}),
                                                  qop(2 * i + 1), S, 0, 0, 0);
    }
    return true;
  };

  // Phase 2: softmax against the wave's reference max and O^T += V^T P'^T.  Returns
  // false (nothing accumulated) when a row's max drifts more than kLazy above it.
  // P' = p * s_V (fp16) is the B operand; V^T comes from LDS by transpose reads as
  // the subnormals c * 2^(2k-24); sum p and sum p * z_V accumulate on the VALU.
  auto pv_tile = [&](const f32x16& S) -> bool {
    wait_lds();
    __builtin_amdgcn_wave_barrier();
    float mx = -INFINITY;
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) mx = fmaxf(mx, S[r2]);
    mx = fmaxf(mx, swap_halves(mx)) * c_score;  // c_score > 0
    // the first fast tile sets the reference max (O, l, z are still zero); the
    // state is uniform across the wave's rows until the slow pass
    const bool first = m_run == -INFINITY;
    if (!first && __any(mx > m_run + kLazy)) return false;
    if (first) m_run = mx;
    const float nm = -m_run;
    u32x4 pb[2];
    float lsum = 0.f, zsum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x4 sv = *(const f32x4*)&s_cst[wave][0][8 * q4 + 4 * g];
      const f32x4 zv = *(const f32x4*)&s_cst[wave][1][8 * q4 + 4 * g];
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const int r0 = 4 * q4 + i;
        // p <= 2^kLazy: no range reduction needed for v_exp_f32
        const float p0 = __builtin_amdgcn_exp2f(fmaf(S[r0], c_score, nm));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(S[r0 + 1], c_score, nm));
        lsum += p0 + p1;
        zsum = fmaf(p0, zv[i], fmaf(p1, zv[i + 1], zsum));
        const f16x2 h = {(_Float16)(p0 * sv[i]), (_Float16)(p1 * sv[i + 1])};
        pb[r0 >> 3][(r0 & 7) >> 1] = __builtin_bit_cast(unsigned, h);
      }
    }
    l_run += lsum;
    z_run += zsum;
    const int G16 = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int row = i16 >> 1, half8 = (i16 & 1) * 8;
      const int tok = pv_tok(s, G16 >> 1, row);
#pragma unroll
      for (int cp = 0; cp < D / 128; ++cp) {
        const int chunk = (D == 256) ? (2 * cp + (G16 & 1)) : (G16 & 1);
        const uint8_t* addr = &s_vcode[wave][tok * C::NB + chunk * 16 + half8];
        i32x2 tr = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) i32x2*)(addr));
        const unsigned x0 = (unsigned)tr[0], x1 = (unsigned)tr[1];
        const unsigned t0w = __builtin_amdgcn_perm(0u, x0, 0x0C010C00u);
        const unsigned t1w = __builtin_amdgcn_perm(0u, x0, 0x0C030C02u);
        const unsigned t2w = __builtin_amdgcn_perm(0u, x1, 0x0C010C00u);
        const unsigned t3w = __builtin_amdgcn_perm(0u, x1, 0x0C030C02u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const unsigned msk = 0x00030003u << (2 * k);
          const u32x4 av = {t0w & msk, t1w & msk, t2w & msk, t3w & msk};
          const int mb = (D == 256) ? 4 * cp + k : k;
          O[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(av), __builtin_bit_cast(f16x8, pb[s]),
                                                         O[mb], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the LDS slots are rewritten by the next tile
    return true;
  };

  // Two register slots hold the packed data of the wave's next tiles: slot A the
  // even tiles, slot B the odd ones.  A slot is refilled (index clamped to the last
  // tile, so every path issues the same loads) as soon as its tile's QK has consumed
  // it, so the next two tiles are in flight while a tile is computed.
  uint32_t slow_bits = 0;  // wave tiles (index i) queued for the slow pass
  {
    for (int i = 0; i < my; i += 2) {
      {
        f32x16 S;
        const bool fast = qk_tile(i, RA, S);
        load_tile(i + 2 < last ? i + 2 : last, RA);
        if (!(fast && pv_tile(S))) slow_bits |= 1u << i;
      }
      const bool second = i + 1 < my;
      f32x16 S;
      bool fast = false;
      if (second) fast = qk_tile(i + 1, RB, S);
      load_tile(i + 3 < last ? i + 3 : last, RB);
      if (second && !(fast && pv_tile(S))) slow_bits |= 2u << i;
    }
  }

  // ---- fast-tile accumulators to value units: O = O * 2^(24-2k) + z
  {
    const float z_row = z_run + swap_halves(z_run);
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b) {
      const float f = ldexpf(1.f, 24 - pv_pos(b));
#pragma unroll
      for (int r = 0; r < 16; ++r) O[b][r] = fmaf(O[b][r], f, z_row);
    }
    z_run = 0.f;
  }

  // ---------------------------------------------------------------- slow tiles
  // Every wave's queued tiles go to one list; waves 0..kSlowWaves-1 take them in
  // turn (a wave may add any tile of the item to its own softmax state: the wave
  // states are merged below).
  if (lane == 0) s_nslow[wave] = __popc(slow_bits);
  __syncthreads();
  int nslow = 0, slot0 = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = s_nslow[w];
    slot0 += w < wave ? c : 0;
    nslow += c;
  }
  for (uint32_t bits = slow_bits; bits; bits &= bits - 1, ++slot0)
    if (lane == 0) s_slow[slot0] = (int16_t)(wave + kWaves * __builtin_ctz(bits));
  __syncthreads();
  uint16_t* s_slowv = (uint16_t*)s_big + (wave % kSlowWaves) * (kTile * C::VROW);
  for (int k = wave; wave < kSlowWaves && k < nslow; k += kSlowWaves) {
    const int j = s_slow[k];
    const int t0 = tile_t0(j);
    const int p = t0 + m;
    const bool hist_tok = p < hist;
    const bool cur_tok = has_new && p < seq && p >= hist;
    int blk, off0, seat0;
    tile_page(j, t0, blk, off0, seat0);
    const int off = off0 + m;
    const uint8_t* ks = kbase + (int64_t)blk * ks0 + (int64_t)off * ks1;
    const uint8_t* vs = vbase + (int64_t)blk * vs0 + (int64_t)off * vs1;
    u32x4 kc[C::NQ], vc[C::NQ];
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) {
      kc[i] = *(const u32x4*)(ks + 32 + g * (D / 8) + 16 * i);
      vc[i] = *(const u32x4*)(vs + g * (D / 8) + 16 * i);
    }
    const u32x2 meta = *(const u32x2*)ks;
    const int64_t own = P.has_stage ? owner[seat0 + off] : -1;
    const bool staged = P.has_stage && hist_tok && own == (int64_t)blk;
    const bool any_st = __any(staged), any_cur = __any(cur_tok);
    // FP32 staged rows of this lane's token (seat row 0 for lanes without one)
    const int64_t seat = staged ? (int64_t)seat0 + off : 0;
    const float* sk_row = P.st.stage_k + (seat * hk + kvh) * D + g * (D / 2);
    const float* sv_row = P.st.stage_v + (seat * hk + kvh) * D + g * (D / 2);
    const int ci = cur_tok ? p - hist : 0;
    unsigned kt_lo, kt_hi, vlo, vhi;
    byte_tables(meta[0], kt_lo, kt_hi);
    value_table(meta[1], vlo, vhi);

    f32x16 S = {};
#pragma unroll
    for (int c0 = 0; c0 < C::NCH; c0 += C::CPR) {
      f32x4 fk[C::CPR][4], fv[C::CPR][4];
      if (any_st) {
#pragma unroll
        for (int cc = 0; cc < C::CPR; ++cc)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            fk[cc][u] = *(const f32x4*)(sk_row + 16 * (c0 + cc) + 4 * u);
            fv[cc][u] = *(const f32x4*)(sv_row + 16 * (c0 + cc) + 4 * u);
          }
      }
#pragma unroll
      for (int cc = 0; cc < C::CPR; ++cc) {
        const int c = c0 + cc;
        unsigned ok[8], ov[8];
        lut16(kc[c >> 2][c & 3], kt_lo, kt_hi, ok);
        table_pairs(vc[c >> 2][c & 3], vlo, vhi, ov);
        if (any_st && staged) {
          // K in the lookup's pair order (e, e+4) / (e+8, e+12); V as (e, e+8)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            ok[k] = hist_pair(fk[cc][0][k], fk[cc][1][k]);
            ok[4 + k] = hist_pair(fk[cc][2][k], fk[cc][3][k]);
          }
#pragma unroll
          for (int k = 0; k < 8; ++k)
            ov[k] = hist_pair(fv[cc][k >> 2][k & 3], fv[cc][2 + (k >> 2)][k & 3]);
        }
        if (any_cur && cur_tok) {
          const uint16_t* kr = &s_cur[0][ci][g * (D / 2) + 16 * c];
          const uint16_t* vr = &s_cur[1][ci][g * (D / 2) + 16 * c];
          kpairs16(*(const u32x4*)kr, *(const u32x4*)(kr + 8), ok);
          interleave8(*(const u32x4*)vr, *(const u32x4*)(vr + 8), ov);
        }
        if (!hist_tok && !cur_tok) {
#pragma unroll
          for (int k = 0; k < 8; ++k) ok[k] = ov[k] = 0u;
        }
        S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{ok[0], ok[1], ok[2], ok[3]}),
                                                    qop(2 * c), S, 0, 0, 0);
        S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{ok[4], ok[5], ok[6], ok[7]}),
                                                    qop(2 * c + 1), S, 0, 0, 0);
        // V values of this token to the buffer, columns permuted so that MFMA row i
        // of output block b reads column 32 b + i (d = pv_d(b, i))
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x2 w = {__builtin_amdgcn_perm(ov[q + 4], ov[q], 0x05040100u),
                           __builtin_amdgcn_perm(ov[q + 4], ov[q], 0x07060302u)};
          *(u32x2*)&s_slowv[m * C::VROW + vbuf_col<D>(g, q, c)] = w;
        }
      }
    }
    wait_lds();
    __builtin_amdgcn_wave_barrier();
    // masked scores
    float xs[16];
    float mx = -INFINITY;
    const int limit = seq - nq + (row_ok ? n / G : 0) + 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tp = t0 + out_tok(r, g);
      const bool vis = row_ok && tp < limit;  // limit <= seq
      xs[r] = vis ? S[r] * c_score : -INFINITY;
      mx = fmaxf(mx, xs[r]);
    }
    mx = fmaxf(mx, swap_halves(mx));
    update_max(mx);
    // P = hi + lo, both bf16
    u32x4 ph[2], pl[2];
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const float p0 = (xs[r] == -INFINITY) ? 0.f : exp2f(xs[r] - m_run);
      const float p1 = (xs[r + 1] == -INFINITY) ? 0.f : exp2f(xs[r + 1] - m_run);
      lsum += p0 + p1;
      const unsigned hb = bf16_pair(p0, p1);
      ph[r >> 3][(r & 7) >> 1] = hb;
      pl[r >> 3][(r & 7) >> 1] = bf16_pair(p0 - __uint_as_float(hb << 16), p1 - __uint_as_float(hb & 0xffff0000u));
    }
    l_run += lsum;
    const int G16 = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bf16x8 va;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = 16 * s + 4 * (G16 >> 1) + 8 * h + (i16 >> 2);
          const uint16_t* addr = &s_slowv[key * C::VROW + 32 * b + 16 * (G16 & 1) + 4 * (i16 & 3)];
          auto t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(addr));
#pragma unroll
          for (int e = 0; e < 4; ++e) va[4 * h + e] = __builtin_bit_cast(__bf16, (unsigned short)t[e]);
        }
        O[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, __builtin_bit_cast(bf16x8, ph[s]), O[b], 0, 0, 0);
        O[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, __builtin_bit_cast(bf16x8, pl[s]), O[b], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- cross-wave merge: common max M and total L per row, then the wave partials
  // are summed in LDS in MFMA register order, two output blocks per round
  const float l_row = l_run + swap_halves(l_run);
  __syncthreads();  // every wave is past its slow tiles (s_big is free)
  if (g == 0) { s_ml[wave][0][m] = m_run; s_ml[wave][1][m] = l_row; }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][0][n]);
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float mw = s_ml[w][0][n];
    if (mw != -INFINITY) L += s_ml[w][1][n] * exp2f(mw - M);
  }
  const float fw = (m_run == -INFINITY || !(L > 0.f)) ? 0.f : exp2f(m_run - M) / L;
  f32x4* buf = (f32x4*)s_big;  // [kWaves][2 blocks][4][64] f32x4
  f32x4* po = (f32x4*)(P.part_o + (int64_t)part * 32 * D);
#pragma unroll
  for (int rb = 0; rb < C::MBLK / 2; ++rb) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x16& Ob = O[2 * rb + bb];
        buf[((wave * 2 + bb) * 4 + q) * 64 + lane] =
            f32x4{Ob[4 * q] * fw, Ob[4 * q + 1] * fw, Ob[4 * q + 2] * fw, Ob[4 * q + 3] * fw};
      }
    __syncthreads();
    f32x4 acc = buf[tid];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) acc += buf[w * kThreads + tid];
    const int e = rb * kThreads + tid;  // f32x4 index of the partial (row = e % 32)
    if ((e & 31) < nrows) po[e] = acc;
    __syncthreads();
  }
  if (tid < 32) {
    float lse = (L > 0.f && M != -INFINITY) ? (M + log2f(L)) * kLn2 : -INFINITY;
    if (M != M || L != L) lse = NAN;
    P.part_lse[(int64_t)part * 32 + tid] = lse;
  }
}

// FP32 LSE merge of a group's items (slab_attention.py:341-356 applied in
// sequence; empty parts contribute nothing).  One wave per (group, 64-vector chunk
// of the register-order partial): lane l owns partial vector chunk * 64 + l, i.e.
// row l % 32, four d values.  Online merge over batches of kBatch items whose
// partial vectors and LSEs are loaded together.
constexpr int kBatch = 40;  // one round of loads for up to 40 items

template <int D>
__global__ __launch_bounds__(64) void attn_merge_kernel(AttnParams P) {
  using C = Cfg<D>;
  const oscar_attn_args_v1& A = P.a;
  // the group record carries everything the merge needs (no dependent loads)
  const int32_t* grp = A.groups + (int64_t)blockIdx.x * OSCAR_GROUP_INTS;
  const int req = grp[0], kvh = grp[1], i0 = grp[2], ni = grp[3], a = grp[4], nq = grp[5];
  (void)req;
  const int G = P.group;
  const int lane = threadIdx.x;
  const int n = lane & 31, gg = lane >> 5;
  const int bq = blockIdx.y, b = bq >> 2, q = bq & 3;
  const int e = bq * 64 + lane;  // f32x4 index in the partial
  const bool row_ok = n < nq * G;
  const f32x4* po = (const f32x4*)P.part_o + (int64_t)i0 * C::NV + e;
  const float* pl = P.part_lse + (int64_t)i0 * 32 + n;
  float M = -INFINITY, L = 0.f;
  bool nan = false;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < ni; i += kBatch) {
    float l[kBatch];
    f32x4 x[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const bool in = i + u < ni;
      l[u] = in ? pl[(int64_t)(i + u) * 32] : -INFINITY;
      x[u] = (in && row_ok) ? po[(int64_t)(i + u) * C::NV] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float mb = -INFINITY;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      nan |= l[u] != l[u];
      mb = fmaxf(mb, l[u]);
    }
    const float Mn = fmaxf(M, mb);
    if (Mn != -INFINITY) {
      const float f = (M == -INFINITY) ? 0.f : expf(M - Mn);
      acc *= f;
      L *= f;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const float w = (l[u] == -INFINITY) ? 0.f : expf(l[u] - Mn);
        L += w;
        acc += (w > 0.f) ? x[u] * w : f32x4{0.f, 0.f, 0.f, 0.f};
      }
      M = Mn;
    }
  }
  if (!row_ok) return;
  float lse = -INFINITY;
  if (nan) {
    acc = f32x4{NAN, NAN, NAN, NAN};
    lse = NAN;
  } else if (M != -INFINITY && L > 0.f) {
    acc *= 1.f / L;
    lse = M + logf(L);
  } else {
    acc = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int tok = a + n / G, head = kvh * G + n % G;
  float* orow = A.out_rot + ((int64_t)tok * A.num_q_heads + head) * D;
#pragma unroll
  for (int j = 0; j < 4; ++j) orow[pv_d<D>(b, out_tok(4 * q + j, gg))] = acc[j];
  if (bq == 0 && gg == 0) A.lse[(int64_t)tok * A.num_q_heads + head] = lse;
}

template <int D>
int launch_decode(const AttnParams& p, hipStream_t s) {
  if (p.a.phases != 2) {
    hipLaunchKernelGGL(attn_main_kernel<D>, dim3(p.a.num_items), dim3(kThreads), 0, s, p);
    OSCAR_CHECK_LAUNCH("attn_main_kernel");
  }
  if (p.a.phases != 1) {
    hipLaunchKernelGGL(attn_merge_kernel<D>, dim3(p.a.num_groups, Cfg<D>::NV / 64), dim3(64), 0, s, p);
    OSCAR_CHECK_LAUNCH("attn_merge_kernel");
  }
  return 0;
}

}  // namespace

}  // namespace oscar

using namespace oscar;

// ----------------------------------------------------------------- planning
extern "C" int oscar_attn_plan_v1(const int32_t* qsl, const int32_t* seqs, int32_t num_reqs,
                                  int32_t has_new, int32_t num_kv_heads, int32_t group,
                                  int32_t head_dim, int32_t chunk_tokens, int32_t target_items,
                                  int32_t* items, int32_t max_items, int32_t* groups,
                                  int32_t max_groups, oscar_plan_v1* plan) {
  if (!qsl || !seqs || !plan || num_reqs < 0 || num_kv_heads < 1 || num_kv_heads > 0xffff || group < 1)
    return fail(-22, "oscar_attn_plan_v1: invalid arguments");
  if (head_dim != 128 && head_dim != 256)
    return fail(-22, "oscar_attn_plan_v1: head_dim %d unsupported (128/256)", head_dim);
  if (chunk_tokens < kTile) chunk_tokens = kTile;
  if (chunk_tokens > kMaxItemTokens) chunk_tokens = kMaxItemTokens;
  if (target_items < 1) target_items = 1;
  // Per (request, kv head) group: body tiles are the full tiles every row sees
  // (before min(history, seq - n_q + 1)); the tiles after them (current chunk,
  // causal boundary, ragged end) form one tail item per group.  Body tiles are
  // dealt to k items round-robin (item j: tiles j, j + k, ...), so a contiguous
  // run of expensive tiles (the FP32 staging window) spreads over many items.
  struct Grp { int req, kvh, nbody, ntail, k, first_slot; };
  int ngroups = 0, ntails = 0;
  int64_t body_total = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int nq = qsl[r + 1] - qsl[r];
    if (nq <= 0) continue;
    if (nq * group > 32) return fail(-22, "oscar_attn_plan_v1: request %d has %d rows > 32", r, nq * group);
    if (seqs[r] < 0 || (has_new && seqs[r] < nq))
      return fail(-22, "oscar_attn_plan_v1: sequence length must cover its query chunk");
    ngroups += num_kv_heads;
    if (ngroups > (1 << 24)) return fail(-22, "oscar_attn_plan_v1: too many request x kv-head groups");
  }
  std::vector<Grp> gl((size_t)(ngroups > 0 ? ngroups : 1));
  int gi = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int nq = qsl[r + 1] - qsl[r];
    if (nq <= 0) continue;
    const int seq = seqs[r], hist = has_new ? seq - nq : seq;
    int fast_end = seq - nq + 1 < hist ? seq - nq + 1 : hist;
    if (fast_end < 0) fast_end = 0;
    const int nbody = fast_end / kTile;
    const int ntail = (seq + kTile - 1) / kTile - nbody;
    for (int h = 0; h < num_kv_heads; ++h) {
      gl[gi++] = {r, h, nbody, ntail, 0, 0};
      body_total += nbody;
      ntails += ntail > 0;
    }
  }
  const int budget = target_items - ntails > ngroups ? target_items - ntails : ngroups;
  const int max_tiles = chunk_tokens / kTile;
  int nitems = 0, max_k = 0;
  for (int q = 0; q < ngroups; ++q) {
    Grp& G = gl[q];
    int k = 0;
    if (G.nbody > 0) {
      k = (int)(((int64_t)G.nbody * budget * 2 + body_total) / (2 * body_total));
      if (k < 1) k = 1;
      if ((G.nbody + k - 1) / k > max_tiles) k = (G.nbody + max_tiles - 1) / max_tiles;
      if (k > G.nbody) k = G.nbody;
    }
    G.k = k;
    G.first_slot = nitems;
    nitems += k + (G.ntail > 0);
    if (k > max_k) max_k = k;
  }
  plan->num_items = nitems;
  plan->num_groups = ngroups;
  plan->partial_bytes = (int64_t)nitems * 32 * (head_dim + 1) * (int64_t)sizeof(float);
  if (items == nullptr || groups == nullptr) return nitems;  // size query
  if (nitems > max_items || ngroups > max_groups) return fail(-28, "oscar_attn_plan_v1: buffers too small");
  // Launch order: the tail items first (they carry the slow work), then the body
  // items interleaved over the groups so that consecutive workgroups, which the
  // hardware deals round-robin to the 8 XCDs, spread every group over the chip.
  // The partial slots of a group stay contiguous (tail, then body) for the merge.
  int idx = 0;
  auto emit = [&](const Grp& G, int slot, int first, int stride, int count) {
    int32_t* it = items + (int64_t)idx++ * OSCAR_WORK_INTS;
    const int nq = qsl[G.req + 1] - qsl[G.req];
    it[0] = G.req;
    it[1] = G.kvh | (nq << 16);
    it[2] = first;
    it[3] = stride;
    it[4] = count;
    it[5] = slot;
    it[6] = qsl[G.req];
    it[7] = seqs[G.req];
  };
  for (int q = 0; q < ngroups; ++q)
    if (gl[q].ntail > 0) emit(gl[q], gl[q].first_slot, gl[q].nbody, 1, gl[q].ntail);
  for (int pos = 0; pos < max_k; ++pos)
    for (int q = 0; q < ngroups; ++q) {
      const Grp& G = gl[q];
      if (pos >= G.k) continue;
      emit(G, G.first_slot + (G.ntail > 0) + pos, pos, G.k, (G.nbody - pos + G.k - 1) / G.k);
    }
  for (int q = 0; q < ngroups; ++q) {
    int32_t* gr = groups + (int64_t)q * OSCAR_GROUP_INTS;
    gr[0] = gl[q].req;
    gr[1] = gl[q].kvh;
    gr[2] = gl[q].first_slot;
    gr[3] = gl[q].k + (gl[q].ntail > 0);
    gr[4] = qsl[gl[q].req];
    gr[5] = qsl[gl[q].req + 1] - qsl[gl[q].req];
    gr[6] = gr[7] = 0;
  }
  return nitems;
}

extern "C" int oscar_attn_decode_v1(const oscar_attn_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_attn_decode_v1: null args");
  const oscar_attn_args_v1& a = *args;
  const int64_t D = a.cache.head_dim;
  if (D != 128 && D != 256) return fail(-22, "oscar_attn_decode_v1: head_dim %lld unsupported", (long long)D);
  if (a.num_items <= 0 || a.num_groups <= 0) return 0;
  if (!a.q || !a.items || !a.groups || !a.workspace || !a.out_rot || !a.lse || !a.block_table ||
      !a.query_start_loc || !a.seq_lens)
    return fail(-22, "oscar_attn_decode_v1: missing pointer");
  if ((a.k_new == nullptr) != (a.v_new == nullptr))
    return fail(-22, "oscar_attn_decode_v1: both new K and V must be supplied together");
  if (a.phases < 0 || a.phases > 2) return fail(-22, "oscar_attn_decode_v1: phases must be 0, 1 or 2");
  if (a.cache.num_kv_heads < 1 || a.num_q_heads % a.cache.num_kv_heads)
    return fail(-22, "oscar_attn_decode_v1: Hq must be a multiple of Hk");
  if ((a.cache.k_stride[2] & 15) || (a.cache.v_stride[2] & 15) || (a.cache.k_stride[1] & 15) ||
      (a.cache.v_stride[1] & 15) || (a.cache.k_stride[0] & 15) || (a.cache.v_stride[0] & 15) ||
      (((uintptr_t)a.cache.k) & 15) || (((uintptr_t)a.cache.v) & 15))
    return fail(-22, "oscar_attn_decode_v1: cache slots must be 16-byte aligned");
  // queries and the current chunk are read as 16-byte vectors
  if ((a.q_stride_token & 7) || (((uintptr_t)a.q) & 15) ||
      (a.k_new && ((a.kv_new_stride_token & 7) || (((uintptr_t)a.k_new) & 15) || (((uintptr_t)a.v_new) & 15))))
    return fail(-22, "oscar_attn_decode_v1: q / k_new / v_new rows must be 16-byte aligned");
  if (a.cache.block_size < kTile || a.cache.block_size % kTile || a.cache.block_size > (1 << 20))
    return fail(-22, "oscar_attn_decode_v1: block_size %lld must be a multiple of %d (<= 2^20)",
                (long long)a.cache.block_size, kTile);
  if (a.staging && (a.staging->rows < 1 || a.staging->rows * a.cache.block_size >= (1ll << 31) ||
                    (((uintptr_t)a.staging->stage_k) & 15) || (((uintptr_t)a.staging->stage_v) & 15)))
    return fail(-22, "oscar_attn_decode_v1: staging arena rows out of range or unaligned");
  AttnParams p{};
  p.a = a;
  p.has_stage = a.staging != nullptr;
  if (a.staging) p.st = *a.staging;
  p.group = (int)(a.num_q_heads / a.cache.num_kv_heads);
  p.part_o = (float*)a.workspace;
  p.part_lse = p.part_o + (int64_t)a.num_items * 32 * D;
  hipStream_t s = (hipStream_t)stream;
  return D == 256 ? launch_decode<256>(p, s) : launch_decode<128>(p, s);
}
