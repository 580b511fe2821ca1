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

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 32;
constexpr int kDepth = 3;            // tiles of packed data in flight per wave
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
  static constexpr int CPR = 2;          // chunks per staged-row load round
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
  __shared__ __attribute__((aligned(16))) uint8_t s_vcode[kWaves][2][kTile * C::NB];  // double buffer
  __shared__ __attribute__((aligned(16))) float s_cst[kWaves][2][2][kTile];
  __shared__ __attribute__((aligned(16))) float s_ml[kWaves][2][32];
  __shared__ __attribute__((aligned(16))) uint16_t s_cur[2][kMaxCur][D];  // current K / V
  __shared__ __attribute__((aligned(16))) u32x4 s_q[C::KSTEPS][64];        // Q^T operand
  // union: slow-tile V values (bf16, permuted columns) / cross-wave merge buffers
  constexpr int kMergeBytes = 2 * C::NV * 16, kSlowBytes = kWaves * kTile * C::VROW * 2;
  __shared__ __attribute__((aligned(16))) uint8_t s_big[kMergeBytes > kSlowBytes ? kMergeBytes : kSlowBytes];
  uint16_t* s_slowv = (uint16_t*)s_big + wave * (kTile * C::VROW);
  const unsigned st_rows = (unsigned)P.st.rows;

  // ---- prologue: page of every item tile, current chunk and queries, loaded together
  bool any_cur_tile = false;
  for (int j = tid; j < count; j += kThreads) {
    const int t0 = tile_t0(j);
    int32_t b = 0;
    if (t0 < hist) {
      b = A.block_table[(int64_t)req * A.block_table_stride + t0 / bs];
      // ids outside the cache are clamped (the host validates tables; this keeps a
      // bad table from faulting)
      b = (b < 0 || b >= A.cache.num_blocks) ? 0 : b;
    }
    s_blk[j] = b;
    s_seat[j] = P.has_stage ? (int)((unsigned)b % st_rows) * bs : 0;
  }
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
  // of the code dwords (elements k, k+8 of each 16-element chunk paired); the Q^T
  // operand of K-step j for lane l lives at s_q[j][l] (shared by the waves)
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
      interleave8(lo, hi, o);
      s_q[2 * c][lane] = u32x4{o[0], o[1], o[2], o[3]};
      s_q[2 * c + 1][lane] = u32x4{o[4], o[5], o[6], o[7]};
    }
  }
  const float c_score = A.scale * kLog2e;  // scores in log2 units
  __syncthreads();
  auto qop = [&](int j) { return __builtin_bit_cast(bf16x8, s_q[j][lane]); };

  // ---- running state (per lane row n): reference max m_run (log2 units), sum l, z
  float m_run = -INFINITY, l_run = 0.f, z_run = 0.f;
  f32x16 O[C::MBLK];
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = 0.f;

  // wave w takes item tiles j = w + 4 i, i < my
  const int my = count > wave ? (count - 1 - wave) / kWaves + 1 : 0;
  uint64_t slow_mask = 0, st_bits = 0;
  const uint8_t* kbase = A.cache.k + (int64_t)kvh * A.cache.k_stride[2];
  const uint8_t* vbase = A.cache.v + (int64_t)kvh * A.cache.v_stride[2];
  const int64_t ks0 = A.cache.k_stride[0], ks1 = A.cache.k_stride[1];
  const int64_t vs0 = A.cache.v_stride[0], vs1 = A.cache.v_stride[1];
  const int64_t* owner = P.st.owner;

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

  // page of item tile j, first key t0 (wave-uniform): block, in-page offset of t0
  // and seat-row base.  Tiles past the history, and the placeholder tile j >= count
  // a wave without tiles loads in the pipeline prologue (its s_blk entry is never
  // written), read block 0 at offsets 0..31 (< block_size).
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
    int off0, seat0;
    tile_page(j, t0, r.blk, off0, seat0);
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

  // ---------------------------------------------------------------- fast tiles
  // Straight-line in the O accumulators (no branch around an MFMA, no VALU on O):
  // a tile that turns out slow (staged token, mask, ragged end, or a max more than
  // kLazy above the wave's reference max) or that only pads the pipeline runs with
  // P = 0 and, if real, is queued for the slow pass.
  //
  // Two tiles are in compute at once: iteration i runs the QK MFMAs of tile i+1
  // (their operands looked up on the VALU in between), then the softmax of tile
  // i+1 on the VALU next to the PV MFMAs of tile i, so the MFMA and VALU pipes
  // overlap.  V codes and V constants sit in LDS double buffers (tile parity).

  // QK of tile ti: V codes and V constants to LDS buffer bf, S^T = K Q^T with the
  // exact history values looked up per code pair.  Returns the pre-softmax slow
  // flag (a staged token, or a tile beyond the fast range).
  auto qk_tile = [&](int ti, const TileRegs<D>& r, int bf, f32x16& S) -> bool {
    const int t0 = tile_t0(wave + kWaves * ti);
    const int p = t0 + m;
    const bool real = ti < my;
    const bool staged = P.has_stage && real && p < hist && r.own == (int64_t)r.blk;
    st_bits |= (uint64_t)staged << (ti & 63);  // ti < 64 whenever staged
    const bool slow = real && !((t0 + kTile <= fast_end) && !__any(staged));
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) *(u32x4*)&s_vcode[wave][bf][m * C::NB + g * (D / 8) + 16 * i] = r.v[i];
    s_cst[wave][bf][0][m] = f16_bits_to_f32(r.meta[1] & 0xffff);  // both halves write the same
    s_cst[wave][bf][1][m] = f16_bits_to_f32(r.meta[1] >> 16);
    unsigned lut_lo, lut_hi;
    value_table(r.meta[0], lut_lo, lut_hi);
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) S[r2] = 0.f;
#pragma unroll
    for (int i = 0; i < C::NCH; ++i) {
      unsigned o[8];
      table_pairs(r.k[i >> 2][i & 3], lut_lo, lut_hi, o);
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]}),
                                                  qop(2 * i), S, 0, 0, 0);
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u32x4{o[4], o[5], o[6], o[7]}),
                                                  qop(2 * i + 1), S, 0, 0, 0);
    }
    return slow;
  };

  // softmax of tile ti (scores S, V constants in buffer bf): P' = p * s_V (fp16)
  // feeds the PV MFMA, sum p and sum p * z_V accumulate on the VALU
  auto softmax_tile = [&](int ti, const f32x16& S, bool slow, int bf, u32x4* pb) {
    const bool real = ti < my;
    wait_lds();
    __builtin_amdgcn_wave_barrier();
    float xs[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) {
      xs[r2] = S[r2] * c_score;
      mx = fmaxf(mx, xs[r2]);
    }
    mx = fmaxf(mx, swap_halves(mx));
    // the first used tile sets the reference max (O, l, z are still zero); after
    // that a tile whose max drifts more than kLazy above it goes to the slow pass
    const bool first = m_run == -INFINITY;  // uniform: fast-tile scores are finite
    slow = slow || (real && !first && __any(mx > m_run + kLazy));
    if (slow) slow_mask |= 1ull << ti;
    const bool use = real && !slow;
    if (use && first) m_run = mx;
    float lsum = 0.f, zsum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x4 sv = *(const f32x4*)&s_cst[wave][bf][0][8 * q4 + 4 * g];
      const f32x4 zv = *(const f32x4*)&s_cst[wave][bf][1][8 * q4 + 4 * g];
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const int r0 = 4 * q4 + i;
        // p <= 2^kLazy: no range reduction needed for v_exp_f32
        const float p0 = use ? __builtin_amdgcn_exp2f(xs[r0] - m_run) : 0.f;
        const float p1 = use ? __builtin_amdgcn_exp2f(xs[r0 + 1] - m_run) : 0.f;
        lsum += p0 + p1;
        zsum = fmaf(p0, zv[i], fmaf(p1, zv[i + 1], zsum));
        const f16x2 h = {(_Float16)(p0 * sv[i]), (_Float16)(p1 * sv[i + 1])};
        pb[r0 >> 3][(r0 & 7) >> 1] = __builtin_bit_cast(unsigned, h);
      }
    }
    l_run += lsum;
    z_run += zsum;
  };

  // PV of a tile whose V codes sit in buffer bf: O^T += V^T P'^T, V^T from LDS via
  // transpose reads
  auto pv_tile = [&](int bf, const u32x4* pb) {
    const int G16 = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int row = i16 >> 1, half8 = (i16 & 1) * 8;
      const int tok = pv_tok(s, G16 >> 1, row);
#pragma unroll
      for (int cp = 0; cp < D / 128; ++cp) {
        const int chunk = (D == 256) ? (2 * cp + (G16 & 1)) : (G16 & 1);
        const uint8_t* addr = &s_vcode[wave][bf][tok * C::NB + chunk * 16 + half8];
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
  };

  // software pipeline: tile t's packed data sits in register slot t % 3 from its load
  // until its QK, then the slot is refilled with tile t + 3 (clamped to the last tile:
  // the surplus loads at the end re-read a tile already in cache and are never used)
  {
    static_assert(kDepth == 3, "the unrolled slot rotation below assumes three slots");
    TileRegs<D> R[kDepth];
    const int last = my > 0 ? my - 1 : 0;
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_tile(d < last ? d : last, R[d]);
    f32x16 S;
    u32x4 pb[2];
    {
      const bool sl = qk_tile(0, R[0], 0, S);
      softmax_tile(0, S, sl, 0, pb);
      load_tile(3 < last ? 3 : last, R[0]);
    }
    for (int base = 0; base < my; base += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const int i = base + d;          // tile whose PV runs now
        const int dn = (d + 1) % kDepth;  // slot of tile i + 1
        f32x16 Sn;
        const bool sl = qk_tile(i + 1, R[dn], (i + 1) & 1, Sn);
        u32x4 pbn[2];
        softmax_tile(i + 1, Sn, sl, (i + 1) & 1, pbn);
        pv_tile(i & 1, pb);
        pb[0] = pbn[0];
        pb[1] = pbn[1];
        load_tile(i + 4 < last ? i + 4 : last, R[dn]);
      }
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
  while (slow_mask) {
    const int ti = __builtin_ctzll(slow_mask);
    slow_mask &= slow_mask - 1;
    const int j = wave + kWaves * ti;
    const int t0 = tile_t0(j);
    const int p = t0 + m;
    const bool staged = (st_bits >> ti) & 1;
    const bool hist_tok = p < hist;
    const bool cur_tok = has_new && p < seq && p >= hist;
    const bool any_st = __any(staged), any_cur = __any(cur_tok);
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
    // FP32 staged rows of this lane's token (seat row 0 for lanes without one)
    const int64_t seat = staged ? (int64_t)seat0 + off : 0;
    const float* sk_row = P.st.stage_k + (seat * hk + kvh) * D + g * (D / 2);
    const float* sv_row = P.st.stage_v + (seat * hk + kvh) * D + g * (D / 2);
    const int ci = cur_tok ? p - hist : 0;
    unsigned klo, khi, vlo, vhi;
    value_table(meta[0], klo, khi);
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
        table_pairs(kc[c >> 2][c & 3], klo, khi, ok);
        table_pairs(vc[c >> 2][c & 3], vlo, vhi, ov);
        if (any_st && staged) {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            ok[k] = hist_pair(fk[cc][k >> 2][k & 3], fk[cc][2 + (k >> 2)][k & 3]);
            ov[k] = hist_pair(fv[cc][k >> 2][k & 3], fv[cc][2 + (k >> 2)][k & 3]);
          }
        }
        if (any_cur && cur_tok) {
          const uint16_t* kr = &s_cur[0][ci][g * (D / 2) + 16 * c];
          const uint16_t* vr = &s_cur[1][ci][g * (D / 2) + 16 * c];
          interleave8(*(const u32x4*)kr, *(const u32x4*)(kr + 8), ok);
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

  // ---- cross-wave merge: common max M and total L per row, then the four wave
  // partials are summed in LDS in MFMA register order (16-byte accesses)
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
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] *= fw;
  f32x4* buf = (f32x4*)s_big;  // [2][MBLK][4][64] f32x4
  auto put = [&](int slot) {
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        buf[((slot * C::MBLK + b) * 4 + q) * 64 + lane] =
            f32x4{O[b][4 * q], O[b][4 * q + 1], O[b][4 * q + 2], O[b][4 * q + 3]};
  };
  if (wave >= 2) put(wave - 2);
  __syncthreads();
  if (wave < 2) {
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = buf[((wave * C::MBLK + b) * 4 + q) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) O[b][4 * q + j] += v[j];
      }
    put(wave);
  }
  __syncthreads();
  // item partial: slot 0 + slot 1, register order, rows < nrows; lse [32]
  f32x4* po = (f32x4*)(P.part_o + (int64_t)part * 32 * D);
  for (int e = tid; e < C::NV; e += kThreads)
    if ((e & 31) < nrows) po[e] = buf[e] + buf[C::NV + e];
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
constexpr int kBatch = 16;

template <int D>
__global__ __launch_bounds__(64) void attn_merge_kernel(AttnParams P) {
  using C = Cfg<D>;
  const oscar_attn_args_v1& A = P.a;
  const int32_t* grp = A.groups + (int64_t)blockIdx.x * 4;
  const int req = grp[0], kvh = grp[1], i0 = grp[2], ni = grp[3];
  const int a = A.query_start_loc[req];
  const int nq = A.query_start_loc[req + 1] - a;
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
    groups[q * 4 + 0] = gl[q].req;
    groups[q * 4 + 1] = gl[q].kvh;
    groups[q * 4 + 2] = gl[q].first_slot;
    groups[q * 4 + 3] = gl[q].k + (gl[q].ntail > 0);
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
