// Streaming split-K paged attention over the packed INT2 history (gfx950).
//
// Replaces oscar_ascend/kernels/slab_attention.py:376-476 (slab_attention) for
// cached requests: decode, MTP verification (1 + 3 drafts x 6 heads = 24 rows),
// cache-only decode, and chunks of more rows (query tokens x heads per KV head) than
// one 32-row MFMA tile holds, which the plan cuts into sub-requests of 32 rows.
// Semantics follow streaming_attention.py:134-196: query i of a request with n_q
// queries and length seq sees keys [0, seq - n_q + i + 1); history keys come from
// the packed cache unless the staging owner tag of their seat equals the physical
// block (then the FP32 staged value is used); keys >= the history length come from
// the current (rotated, unquantized) chunk.
//
// Work decomposition: the host plan (oscar_attn_plan_v1) deals the 32-token key
// tiles of every (request, kv-head) group round-robin to items, the expected staging
// window and slow tail in items of their own, under a bound on the item cost.  One
// 512-thread workgroup (8 waves, two per SIMD) per item; wave w starts with item
// tiles w and w + 8 and then takes the next fast tile from a shared counter.
// Pages hold a multiple of 32 tokens, so a tile never straddles a page: its block
// id, seat row and in-page offset are wave-uniform scalars.  The eight wave
// partials are merged in LDS and the item partial (normalised O in MFMA register
// order, natural-log LSE) goes to the workspace with coalesced 16-byte stores;
// attn_merge_kernel combines the items of each group (FP32 LSE merge,
// slab_attention.py:341-356) into out_rot / lse.
//
// Prologue: the item record, then one round of loads for the page ids (lane i of a
// wave: the wave's tile i) and the queries, then the first two tiles of every wave
// and the owner tags of all its tiles.  The tags give each tile's staged-token mask
// (owner tag == block); tiles with a staged token or past the fast range (current
// chunk, causal boundary, ragged end) form the slow set.
//
// Fast tiles (INT2 history only, no staged token, no mask; one wave, 32 tokens x 32
// rows, S^T = K Q^T then O^T += V^T P^T), with the next two tiles of the wave in
// flight in two register slots:
//  * QK (bf16 MFMA 32x32x16): the K operand holds exactly the reference's history
//    values bf16(fp16(code*scale + zero)).  A token has only four of them; they form
//    byte tables and v_perm_b32 lookups turn 4 codes into 4 values, so scores and
//    LSE carry the reference rounding.
//  * PV (fp16 MFMA): V codes go to LDS in their natural layout and come back
//    transposed with ds_read_b64_tr_b8 (8 tokens x 1 byte = 4 codes per lane); one
//    v_perm and one AND per fp16 pair give the subnormal c*2^(2k-24) for code bits
//    2k..2k+1, the B operand is P' = p*s_V (fp16, round to nearest) and
//    sum_t p*z_V accumulates on the VALU.
//  * softmax against a lazy reference max per row: it moves (rescaling O, l, z) only
//    when a tile's max exceeds it by more than kLazy, so p <= 2^kLazy.
//
// Slow tiles run after the fast tiles, one at a time by the whole workgroup: every
// thread loads its share of the tile (staged FP32 values, codes or current chunk)
// into registers one tile ahead, all threads build the tile's K operands and V
// values in LDS (rounded as the reference does), and one wave adds the tile to its
// softmax state with P split into bf16 hi + lo parts while the next tile's loads
// are in flight.
#include <mutex>
#include <vector>

#include "common.h"
#include "store_quant.h"

namespace oscar {

namespace {

constexpr int kWaves = 8;            // two waves per SIMD
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 32;
constexpr int kMaxItemTokens = 8192; // keys per item (32 tiles per wave)
constexpr int kMaxPages = kMaxItemTokens / kTile + 2;
constexpr int kMaxStride = 0xfff;     // item record: tile stride in bits 0-11 of word 3
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazy = 8.f;         // max drift (log2 units) before O is rescaled
// largest V scale (after the wave's power-of-two factor) in the fast PV operand:
// P' = p * s_V with p <= 2^kLazy stays below the fp16 maximum 65504
constexpr float kVScaleMax = 255.f;
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

// 16-byte store of element `index` of a (wave-uniform) f32x4 array, written past
// this XCD's L2 (buffer_store_dwordx4 with the sc1 cache policy): the item partials
// are read by the merge launch from other XCDs anyway, and written this way they leave
// no dirty L2 lines for the end of the launch to write back (measured: 0.6 us less per
// config-4a step, 1.3 us at one request).  One 16-byte store per lane keeps the
// memory writes at the payload (two 8-byte stores doubled WRITE_SIZE).
__device__ __forceinline__ void store_through(f32x4* base, int index, f32x4 v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, index * 16, 0, 16 /* sc1 */);
}

// Query dtype QT (OSCAR_BF16 or OSCAR_F16): the dtype of the QK operands, of the
// slow tiles' V values and of P in their PV.
//
// reference history rounding q_dtype(fp16(x)) (streaming_attention.py:124) of a pair
// (a -> low half, b -> high half) with the packed RNE conversions v_cvt_pk_f16_f32
// (/ v_cvt_f32_f16 / v_cvt_pk_bf16_f32 for bf16 queries)
template <int QT>
__device__ __forceinline__ unsigned hist_pair(float a, float b) {
  const f16x2 h = __builtin_convertvector(f32x2{a, b}, f16x2);
  if constexpr (QT == OSCAR_F16) {
    return __builtin_bit_cast(unsigned, h);
  } else {
    const f32x2 w = __builtin_convertvector(h, f32x2);
    return __builtin_bit_cast(unsigned, __builtin_convertvector(w, bf16x2));
  }
}
// pair (RNE) of two floats in the query dtype, and the value of its half k
template <int QT>
__device__ __forceinline__ unsigned q_pair(float a, float b) {
  if constexpr (QT == OSCAR_F16) return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a, b}, f16x2));
  else return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <int QT>
__device__ __forceinline__ float q_half(unsigned pair, int k) {
  const unsigned bits = k ? pair >> 16 : pair & 0xffffu;
  if constexpr (QT == OSCAR_F16) return f16_bits_to_f32(bits);
  else return __uint_as_float(bits << 16);
}
// 8 query-dtype elements (one MFMA operand per lane)
template <int QT> struct QVec { typedef bf16x8 type; };
template <> struct QVec<OSCAR_F16> { typedef f16x8 type; };
// C += A B (32x32x16 MFMA) with operands in the query dtype, given as packed words
template <int QT>
__device__ __forceinline__ f32x16 mma16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (QT == OSCAR_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
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

// history value table of one token, q_dtype(fp16(c*scale + zero)) for c = 0..3
template <int QT>
__device__ __forceinline__ void value_table(unsigned scale_zero, unsigned& lo, unsigned& hi) {
  const float s = f16_bits_to_f32(scale_zero & 0xffff), z = f16_bits_to_f32(scale_zero >> 16);
  float v[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(__fmul_rn((float)c, s), z);  // mul, then add
  lo = hist_pair<QT>(v[0], v[1]);
  hi = hist_pair<QT>(v[2], v[3]);
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

// the four history values of a token as byte tables: t_lo = low bytes of the 16-bit
// values for codes 0..3, t_hi = their high bytes
template <int QT>
__device__ __forceinline__ void byte_tables(unsigned scale_zero, unsigned& t_lo, unsigned& t_hi) {
  unsigned lo, hi;
  value_table<QT>(scale_zero, lo, hi);
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
  int blk;              // physical block of the tile (0 off the history)
};

template <int D, int QT>
__global__ __launch_bounds__(kThreads, 1) void attn_main_kernel(AttnParams P) {
  using C = Cfg<D>;
  using QV = typename QVec<QT>::type;  // one MFMA operand in the query dtype
  const oscar_attn_args_v1& A = P.a;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = lane & 31, g = lane >> 5;
  // item record: request, kv head | query count << 16, tiles first + stride * j for
  // j < count (32 keys each), partial slot, the request's first query token and length
  const int32_t* it = A.items + (int64_t)blockIdx.x * OSCAR_WORK_INTS;
  const int req = it[0], kvh = it[1] & 0xffff, nq = it[1] >> 16;
  const int first = it[2], stride = it[3] & kMaxStride, off = it[3] >> 12, count = it[4], part = it[5];
  const int qa = it[6], seq = it[7];
  const int G = P.group;
  const bool has_new = A.k_new != nullptr;
  // keys [hist, seq) are the current chunk's; this (sub-)request's queries start at
  // offset `off` of the chunk, whose first token is qa - off
  const int hist = has_new ? seq - nq - off : seq;
  const int cur0 = qa - off;
  const int nrows = nq * G;
  const int bs = (int)A.cache.block_size;  // a multiple of 32
  const int64_t hk = A.cache.num_kv_heads;
  if (part < 0 || part >= A.num_items) return;
  // an item that breaks oscar_attn_plan_v1's rules, or whose history needs a block-table
  // column past block_table_cols, poisons its partial (NaN LSE, so the merged rows are
  // NaN) instead of reading out of bounds
  if (req < 0 || req >= A.num_reqs || kvh >= hk || nq < 1 || nrows > 32 || hist < 0 || off < 0 ||
      cur0 < 0 || qa + nq > A.num_tokens || first < 0 || stride < 1 || count < 0 ||
      count > kMaxItemTokens / kTile ||
      (count > 0 && (first + (int64_t)stride * (count - 1)) * kTile >= seq) ||
      (hist > 0 && (hist - 1) / bs >= A.block_table_cols)) {
    if (tid < 32) P.part_lse[(int64_t)part * 32 + tid] = NAN;
    return;
  }
  const int lim0 = seq - nq + 1;                              // first key masked for a row
  const int fast_end = hist < lim0 ? hist : lim0;             // fast tiles end at or before
  auto tile_t0 = [&](int j) { return (first + stride * j) * kTile; };  // first key of item tile j

  // LDS
  __shared__ int32_t s_blk[kMaxPages];                 // block ids of the item's pages
  __shared__ int32_t s_seat[kMaxPages];                // their seat-row base (blk % rows) * bs
  __shared__ __attribute__((aligned(16))) float s_cst[kWaves][2][kTile];
  __shared__ __attribute__((aligned(16))) float s_ml[kWaves][2][32];
  __shared__ __attribute__((aligned(16))) u32x4 s_q[C::KSTEPS][64];        // Q^T operand
  __shared__ uint64_t s_slowset[kMaxItemTokens / kTile / 64];  // slow-set bits of the item tiles
  __shared__ int s_next;                               // next item tile for the fast loop
  __shared__ int16_t s_slow[kMaxItemTokens / kTile];             // the slow tiles, ascending
  __shared__ uint32_t s_tmask[kMaxItemTokens / kTile]; // staged-token mask of every item tile
  // union of the phases: V codes of each wave's current fast tile [kWaves][kTile * NB];
  // the slow tile's K operands (bf16 pairs in MFMA order) [kTile][2][NCH][8] and V
  // values (bf16, permuted columns) [kTile][VROW]; the cross-wave merge rounds of four
  // output blocks [kWaves][4][4][64] f32x4
  constexpr int kVcodeBytes = kWaves * kTile * C::NB;
  constexpr int kKopBytes = kTile * 2 * C::NCH * 8 * 4;
  constexpr int kSlowBytes = kKopBytes + kTile * C::VROW * 2;
  constexpr int kMergeBytes = kWaves * 4 * 4 * 64 * 16;
  constexpr int kU0 = kVcodeBytes > kSlowBytes ? kVcodeBytes : kSlowBytes;
  __shared__ __attribute__((aligned(16))) uint8_t s_u[kU0 > kMergeBytes ? kU0 : kMergeBytes];
  uint8_t (*s_vcode)[kTile * C::NB] = (uint8_t (*)[kTile * C::NB])s_u;
  const unsigned st_rows = (unsigned)P.st.rows;

  // prologue share of wave w: item tiles j = w + kWaves * i, i < my (my <= 32), whose
  // pages, owner tags and (the first two) data it loads
  const int my = count > wave ? (count - 1 - wave) / kWaves + 1 : 0;
  const uint8_t* kbase = A.cache.k + (int64_t)kvh * A.cache.k_stride[2];
  const uint8_t* vbase = A.cache.v + (int64_t)kvh * A.cache.v_stride[2];
  const int64_t ks0 = A.cache.k_stride[0], ks1 = A.cache.k_stride[1];
  const int64_t vs0 = A.cache.v_stride[0], vs1 = A.cache.v_stride[1];

  // ---- prologue.  Three rounds of global loads, issued so that no wait queues
  // behind a later round: (1) lane i < my of each wave loads the page of the wave's
  // tile i (kept in a register for the fast pass, and in LDS for the slow pass, which
  // may run the tile on another wave) and wave 0 loads the queries; (2) once the
  // pages are in, the first two tiles of every wave; (3) the queries go to LDS while
  // the tiles are in flight.
  int wblk = 0, wseat = 0;
  if (lane < my) {
    const int t0 = tile_t0(wave + kWaves * lane);
    if (t0 < hist) wblk = A.block_table[(int64_t)req * A.block_table_stride + t0 / bs];
  }
  const int n = m;
  const bool row_ok = n < nrows;
  u32x4 qv[2 * C::NCH];
  if (wave == 0) {
    const int qtok = qa + (row_ok ? n / G : 0);
    const int qhead = kvh * G + (row_ok ? n % G : 0);
    const uint16_t* qrow = (const uint16_t*)A.q + (int64_t)qtok * A.q_stride_token + (int64_t)qhead * D + g * (D / 2);
#pragma unroll
    for (int c = 0; c < 2 * C::NCH; ++c) qv[c] = *(const u32x4*)(qrow + 8 * c);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep round 1 ahead of round 2
  if (lane < my) {
    // ids outside the cache are clamped (a table entry may hold any value; this keeps
    // a bad one from faulting)
    wblk = (wblk < 0 || wblk >= A.cache.num_blocks) ? 0 : wblk;
    wseat = P.has_stage ? (int)((unsigned)wblk % st_rows) * bs : 0;
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
    const int off = off0 + m;
    const uint8_t* ks = kbase + (int64_t)r.blk * ks0 + (int64_t)off * ks1;
    const uint8_t* vs = vbase + (int64_t)r.blk * vs0 + (int64_t)off * vs1;
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) {
      r.k[i] = *(const u32x4*)(ks + 32 + g * (D / 8) + 16 * i);
      r.v[i] = *(const u32x4*)(vs + g * (D / 8) + 16 * i);
    }
    r.meta = *(const u32x2*)ks;
  };

  // round 2: the wave's first two tiles (register slots A and B, see the main loop)
  // and the owner tags of the wave's tiles (lanes 0-31 the even tiles, 32-63 the
  // odd ones), whose low words decide (tags are -1 or block ids < 2^31)
  const int last = my > 0 ? my - 1 : 0;
  TileRegs<D> RA, RB;
  load_tile(0, RA);
  load_tile(1 < last ? 1 : last, RB);
  constexpr int kTagRounds = kMaxItemTokens / kTile / kWaves / 2;  // 16
  int32_t tag[kTagRounds];
  {
    const int32_t* own32 = (const int32_t*)P.st.owner;
#pragma unroll
    for (int ii = 0; ii < kTagRounds; ++ii) {
      tag[ii] = -1;
      if (2 * ii < my) {
        const int i = 2 * ii + g;
        const int seat = __builtin_amdgcn_readlane(wseat, 2 * ii + 1 < my ? 2 * ii + 1 : 2 * ii);
        const int seat_e = __builtin_amdgcn_readlane(wseat, 2 * ii);
        const int t0 = tile_t0(wave + kWaves * i);
        if (P.has_stage && i < my && t0 < hist) tag[ii] = own32[2 * ((int64_t)(g ? seat : seat_e) + t0 % bs + m)];
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // round 2 goes out before the LDS writes wait for round 1

  if (lane < my) {
    const int j = wave + kWaves * lane;
    s_blk[j] = wblk;
    s_seat[j] = wseat;
  }
  // queries: lane (row n = m, half g) holds q[n][g*D/2 .. +D/2) in the K-step order
  // of the code lookup (kpairs16); the Q^T operand of K-step j for lane l lives at
  // s_q[j][l] (shared by the waves)
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
      u32x4 lo = qv[2 * c], hi = qv[2 * c + 1];
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
  auto qop = [&](int j) { return __builtin_bit_cast(QV, *(const volatile u32x4*)&s_q[j][lane]); };

  // ---- running state (per lane row n): reference max m_run (log2 units), sum l, z
  float m_run = -INFINITY, l_run = 0.f, z_run = 0.f;
  // Power-of-two factor applied to the V scales of the fast PV operand P' = p * s_V * v_fac
  // (wave-uniform).  p <= 2^kLazy, so P' stays finite in fp16 while s_V * v_fac <=
  // kVScaleMax; a tile whose V scale exceeds that lowers v_fac (and rescales O by the
  // same factor) before its PV.  v_fac = 1 unless some V range exceeds ~765.
  float v_fac = 1.f;
  f32x16 O[C::MBLK];
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = 0.f;

  // Lazy: the reference max of a row only moves when a tile's max exceeds it by
  // more than kLazy (log2 units), so probabilities stay <= 2^kLazy and the O
  // accumulators are touched by the VALU only then.
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

  // ---------------------------------------------------------------- slow tiles
  // The slow set: tiles with a staged token (owner tag == block, from the tags
  // loaded in the prologue) or past the fast range (current chunk, causal
  // boundary, ragged end).  The fast tiles skip them; they run after the fast
  // tiles, one at a time by the whole workgroup: (1) every thread loads the staged
  // FP32 values, codes and constants or current-chunk values of its share (token
  // tid / 16) into registers, one tile ahead; (2) the threads build the tile's K
  // operands and V values into LDS with the reference rounding; (3) one wave
  // (round-robin) adds the tile to its softmax state (the wave states are merged at
  // the end).
#pragma unroll
  for (int ii = 0; ii < kTagRounds; ++ii) {
    if (2 * ii >= my) break;
    const int i = 2 * ii + g, j = wave + kWaves * i;
    const int blk_e = __builtin_amdgcn_readlane(wblk, 2 * ii);
    const int blk_o = __builtin_amdgcn_readlane(wblk, 2 * ii + 1 < my ? 2 * ii + 1 : 2 * ii);
    const bool staged = i < my && tile_t0(j) + m < hist && tag[ii] == (g ? blk_o : blk_e);
    const uint64_t b = __ballot(staged);
    if (lane == 0) {
      s_tmask[wave + kWaves * 2 * ii] = (uint32_t)b;
      if (2 * ii + 1 < my) s_tmask[wave + kWaves * (2 * ii + 1)] = (uint32_t)(b >> 32);
    }
  }
  __syncthreads();
  if (wave < (kMaxItemTokens / kTile) / 64) {
    const int j = 64 * wave + lane;
    const bool slow = j < count && (s_tmask[j] != 0 || tile_t0(j) + kTile > fast_end);
    const uint64_t b = __ballot(slow);
    if (lane == 0) s_slowset[wave] = b;
  }
  __syncthreads();
  // the slow list (ascending tile order)
  int nslow = 0;
#pragma unroll
  for (int w = 0; w < (kMaxItemTokens / kTile) / 64; ++w) {
    const uint64_t word = s_slowset[w];
    if (tid >> 6 == w && ((word >> lane) & 1ull)) s_slow[nslow + __popcll(word & ((1ull << lane) - 1ull))] = (int16_t)tid;
    nslow += __popcll(word);
  }
  nslow = __builtin_amdgcn_readfirstlane(nslow);
  if (tid == 0) s_next = 2 * kWaves;  // the tiles after every wave's first two
  __syncthreads();
  u32x4* s_kop = (u32x4*)s_u;                                 // [kTile][2][NCH][2]
  uint16_t* s_slowv = (uint16_t*)(s_u + kKopBytes);           // [kTile][VROW]
  // builder share: token bt of the tile, units uid = bpart + 16 u (u < NU) of the
  // 4 * NCH (K|V, half, 16-element chunk) units of the token
  constexpr int NU = C::NCH / 4;
  const int bt = tid >> 4, bpart = tid & 15;
  // A slow tile's inputs, per thread (token bt, units u < NU): the staged FP32
  // values (4 x 16 bytes per unit), or the codes (one word per unit, constants in
  // meta), or the current chunk's bf16 values (lo / hi 16 bytes per unit in x[u][0..1])
  // -- loaded into registers one tile ahead, so the next tile's loads are in flight
  // while the runner wave computes the current one.
  f32x4 sx[NU][4];
  u32x2 smeta = {0u, 0u};
  auto slow_flags = [&](int j, bool& b_staged, bool& b_codes, bool& b_cur) {
    const int bp = tile_t0(j) + bt;
    b_staged = (s_tmask[j] >> bt) & 1u;
    b_codes = bp < hist && !b_staged;
    b_cur = has_new && bp >= hist && bp < seq;
  };
  auto load_slow = [&](int j) {
    const int t0 = tile_t0(j);
    int blk, off0, seat0;
    tile_page(j, t0, blk, off0, seat0);
    bool b_staged, b_codes, b_cur;
    slow_flags(j, b_staged, b_codes, b_cur);
    const int bp = t0 + bt;
    const uint8_t* ks = kbase + (int64_t)blk * ks0 + (int64_t)(off0 + bt) * ks1;
    const uint8_t* vs = vbase + (int64_t)blk * vs0 + (int64_t)(off0 + bt) * vs1;
    const int64_t cur_off = (int64_t)(cur0 + (b_cur ? bp - hist : 0)) * A.kv_new_stride_token + (int64_t)kvh * D;
    const int64_t seat_row = ((int64_t)seat0 + off0 + bt) * hk + kvh;  // staged row of the token
    smeta = b_codes ? *(const u32x2*)ks : u32x2{0u, 0u};
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int uid = bpart + 16 * u, kv = uid / (2 * C::NCH), hg = (uid / C::NCH) & 1, c = uid % C::NCH;
      if (b_staged) {
        const f32x4* src = (const f32x4*)((kv ? P.st.stage_v : P.st.stage_k) + seat_row * D + hg * (D / 2) + 16 * c);
#pragma unroll
        for (int x = 0; x < 4; ++x) sx[u][x] = src[x];
      } else if (b_codes) {
        sx[u][0][0] = __uint_as_float(*(const uint32_t*)((kv ? vs : ks + 32) + hg * (D / 8) + 4 * c));
      } else if (b_cur) {
        const uint16_t* src = (const uint16_t*)(kv ? A.v_new : A.k_new) + cur_off + hg * (D / 2) + 16 * c;
        sx[u][0] = __builtin_bit_cast(f32x4, *(const u32x4*)src);
        sx[u][1] = __builtin_bit_cast(f32x4, *(const u32x4*)(src + 8));
      }
    }
  };
  // slow tile j (its inputs loaded by load_slow): every thread builds its units' K
  // operands and V values into LDS with the reference rounding
  auto build_slow = [&](int j) {
    bool b_staged, b_codes, b_cur;
    slow_flags(j, b_staged, b_codes, b_cur);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int uid = bpart + 16 * u, kv = uid / (2 * C::NCH), hg = (uid / C::NCH) & 1, c = uid % C::NCH;
      unsigned o[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
      if (b_staged) {
        const f32x4* f = sx[u];
        if (kv == 0) {
          // K operand pairs in the lookup's order (e, e+4) / (e+8, e+12)
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            o[x] = hist_pair<QT>(f[0][x], f[1][x]);
            o[4 + x] = hist_pair<QT>(f[2][x], f[3][x]);
          }
        } else {
#pragma unroll
          for (int x = 0; x < 8; ++x) o[x] = hist_pair<QT>(f[x >> 2][x & 3], f[2 + (x >> 2)][x & 3]);
        }
      } else if (kv == 0) {
        if (b_cur) {
          kpairs16(__builtin_bit_cast(u32x4, sx[u][0]), __builtin_bit_cast(u32x4, sx[u][1]), o);
        } else if (b_codes) {
          unsigned t_lo, t_hi;
          byte_tables<QT>(smeta[0], t_lo, t_hi);
          lut16(__float_as_uint(sx[u][0][0]), t_lo, t_hi, o);
        }
      } else {
        // V values as (e, e+8) pairs
        if (b_cur) {
          interleave8(__builtin_bit_cast(u32x4, sx[u][0]), __builtin_bit_cast(u32x4, sx[u][1]), o);
        } else if (b_codes) {
          unsigned vlo, vhi;
          value_table<QT>(smeta[1], vlo, vhi);
          table_pairs(__float_as_uint(sx[u][0][0]), vlo, vhi, o);
        }
      }
      if (kv == 0) {
        u32x4* dst = s_kop + ((bt * 2 + hg) * C::NCH + c) * 2;
        dst[0] = u32x4{o[0], o[1], o[2], o[3]};
        dst[1] = u32x4{o[4], o[5], o[6], o[7]};
      } else {
        // to the V buffer, columns permuted so that MFMA row i of output block b
        // reads column 32 b + i (d = pv_d(b, i))
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x2 w = {__builtin_amdgcn_perm(o[q + 4], o[q], 0x05040100u),
                           __builtin_amdgcn_perm(o[q + 4], o[q], 0x07060302u)};
          *(u32x2*)&s_slowv[bt * C::VROW + vbuf_col<D>(hg, q, c)] = w;
        }
      }
    }
  };
  // wave `runner` adds slow tile j (built in LDS) to its softmax state
  auto compute_slow = [&](int j, int runner) {
      const int t0 = tile_t0(j);
      if (wave == runner) {
        f32x16 S = {};
#pragma unroll
        for (int c = 0; c < C::NCH; ++c) {
          const u32x4* src = s_kop + ((m * 2 + g) * C::NCH + c) * 2;
          if constexpr (QT == OSCAR_F16) {
            S = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(QV, src[0]), qop(2 * c), S, 0, 0, 0);
            S = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(QV, src[1]), qop(2 * c + 1), S, 0, 0, 0);
          } else {
            S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(QV, src[0]), qop(2 * c), S, 0, 0, 0);
            S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(QV, src[1]), qop(2 * c + 1), S, 0, 0, 0);
          }
        }
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
        // P = hi + lo, both in the query dtype
        u32x4 ph[2], pl[2];
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = (xs[r] == -INFINITY) ? 0.f : exp2f(xs[r] - m_run);
          const float p1 = (xs[r + 1] == -INFINITY) ? 0.f : exp2f(xs[r + 1] - m_run);
          lsum += p0 + p1;
          const unsigned hb = q_pair<QT>(p0, p1);
          ph[r >> 3][(r & 7) >> 1] = hb;
          pl[r >> 3][(r & 7) >> 1] = q_pair<QT>(p0 - q_half<QT>(hb, 0), p1 - q_half<QT>(hb, 1));
        }
        l_run += lsum;
        const int G16 = lane >> 4, i16 = lane & 15;
#pragma unroll
        for (int b = 0; b < C::MBLK; ++b) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            u32x4 va;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int key = 16 * s + 4 * (G16 >> 1) + 8 * h + (i16 >> 2);
              const uint16_t* addr = &s_slowv[key * C::VROW + 32 * b + 16 * (G16 & 1) + 4 * (i16 & 3)];
              const u32x2 t = __builtin_bit_cast(
                  u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(addr)));
              va[2 * h] = t[0];
              va[2 * h + 1] = t[1];
            }
            O[b] = mma16<QT>(va, ph[s], O[b]);
            O[b] = mma16<QT>(va, pl[s], O[b]);
          }
        }
      }
  };

  // ---------------------------------------------------------------- fast tiles
  // Phase 1 (QK) of a fast tile (INT2 history only, no staged token, no mask): its
  // V codes and V constants go to this wave's LDS slots and S^T = K Q^T runs with
  // the exact history values looked up per code.
  auto qk_tile = [&](const TileRegs<D>& r, f32x16& S) {
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) *(u32x4*)&s_vcode[wave][m * C::NB + g * (D / 8) + 16 * i] = r.v[i];
    const float sv_raw = f16_bits_to_f32(r.meta[1] & 0xffff);
    if (__any(sv_raw * v_fac > kVScaleMax)) {
      // lower v_fac to the largest power of two that keeps every V scale of the tile
      // within kVScaleMax (frexp: mx / kVScaleMax = f * 2^e, f in [0.5, 1))
      int e;
      frexpf(wave_max(sv_raw) / kVScaleMax, &e);
      const float nf = ldexpf(1.f, -e);
      const float f = nf / v_fac;
#pragma unroll
      for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
        for (int r2 = 0; r2 < 16; ++r2) O[b][r2] *= f;
      v_fac = nf;
    }
    s_cst[wave][0][m] = sv_raw * v_fac;  // both halves write the same
    s_cst[wave][1][m] = f16_bits_to_f32(r.meta[1] >> 16);
    unsigned t_lo, t_hi;
    byte_tables<QT>(r.meta[0], t_lo, t_hi);
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) S[r2] = 0.f;
#pragma unroll
    for (int i = 0; i < C::NCH; ++i) {
      unsigned o[8];
      lut16(r.k[i >> 2][i & 3], t_lo, t_hi, o);
      if constexpr (QT == OSCAR_F16) {
        S = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(QV, u32x4{o[0], o[1], o[2], o[3]}), qop(2 * i), S, 0, 0, 0);
        S = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(QV, u32x4{o[4], o[5], o[6], o[7]}), qop(2 * i + 1), S, 0, 0, 0);
      } else {
        S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(QV, u32x4{o[0], o[1], o[2], o[3]}), qop(2 * i), S, 0, 0, 0);
        S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(QV, u32x4{o[4], o[5], o[6], o[7]}), qop(2 * i + 1), S, 0, 0,
                                                    0);
      }
    }
  };

  // Phase 2: softmax against the wave's reference max (moved, with O, l and z
  // rescaled, only when a row's max drifts more than kLazy above it) and
  // O^T += V^T P'^T.
  // P' = p * s_V (fp16) is the B operand; V^T comes from LDS by transpose reads as
  // the subnormals c * 2^(2k-24); sum p and sum p * z_V accumulate on the VALU.
  auto pv_tile = [&](const f32x16& S) {
    wait_lds();
    __builtin_amdgcn_wave_barrier();
    float mx = -INFINITY;
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) mx = fmaxf(mx, S[r2]);
    mx = fmaxf(mx, swap_halves(mx)) * c_score;  // c_score > 0
    update_max(mx);
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
  };

  // Two register slots hold the packed data of the wave's next two tiles.  The
  // first two of a wave are its item tiles w and w + kWaves (loaded in the
  // prologue); after that a wave takes the next fast tile from the shared counter
  // s_next (slow tiles are passed over), so that the waves of the item finish
  // together however their loads are served.  A slot is refilled as soon as its
  // tile's QK has consumed it (with a placeholder load once the tiles run out, so
  // every path issues the same loads), so the next two tiles are in flight while a
  // tile is computed.  A slow tile among the first two is refilled without compute.
  auto slow_bit = [&](int j) { return ((s_slowset[j >> 6] >> (j & 63)) & 1ull) != 0; };
  auto take = [&]() {
    int j;
    do {
      int v = 0;
      if (lane == 0) v = atomicAdd(&s_next, 1);
      j = __builtin_amdgcn_readfirstlane(v);
    } while (j < count && slow_bit(j));
    return j < count ? j : count;
  };
  // page of item tile j (j >= count: the placeholder, block 0 at offsets 0..31)
  auto load_next = [&](int j, TileRegs<D>& r) {
    const bool real = j < count;
    const int off0 = real ? tile_t0(j) % bs : 0;
    r.blk = real ? __builtin_amdgcn_readfirstlane(s_blk[j]) : 0;
    const int off = off0 + m;
    const uint8_t* ks = kbase + (int64_t)r.blk * ks0 + (int64_t)off * ks1;
    const uint8_t* vs = vbase + (int64_t)r.blk * vs0 + (int64_t)off * vs1;
#pragma unroll
    for (int i = 0; i < C::NQ; ++i) {
      r.k[i] = *(const u32x4*)(ks + 32 + g * (D / 8) + 16 * i);
      r.v[i] = *(const u32x4*)(vs + g * (D / 8) + 16 * i);
    }
    r.meta = *(const u32x2*)ks;
  };
  int jA = my > 0 ? wave : count;
  int jB = my > 1 ? wave + kWaves : count;
  while (jA < count || jB < count) {
    {
      const bool fast = jA < count && !slow_bit(jA);
      f32x16 S;
      if (fast) qk_tile(RA, S);
      jA = take();
      load_next(jA, RA);
      if (fast) pv_tile(S);
    }
    const bool fast = jB < count && !slow_bit(jB);
    f32x16 S;
    if (fast) qk_tile(RB, S);
    jB = take();
    load_next(jB, RB);
    if (fast) pv_tile(S);
  }

  // ---- fast-tile accumulators to value units: O = O * 2^(24-2k) / v_fac + z
  {
    const float z_row = z_run + swap_halves(z_run);
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b) {
      const float f = ldexpf(1.f, 24 - pv_pos(b)) / v_fac;
#pragma unroll
      for (int r = 0; r < 16; ++r) O[b][r] = fmaf(O[b][r], f, z_row);
    }
    z_run = 0.f;
  }

  // ---- slow tiles, in value units, one at a time by the whole workgroup: build
  // (all threads), then the next tile's loads go out while one wave computes.  The
  // build buffers alias every wave's V-code slot of the fast loop, so the first build
  // waits until all waves are past it (nslow is the same for the whole workgroup).
  if (nslow > 0) {
    load_slow(__builtin_amdgcn_readfirstlane(s_slow[0]));
    __syncthreads();
  }
#pragma unroll 1
  for (int k = 0; k < nslow; ++k) {
    const int j = __builtin_amdgcn_readfirstlane(s_slow[k]);
    build_slow(j);
    __syncthreads();  // the tile's K operands and V values are in LDS
    if (k + 1 < nslow) load_slow(__builtin_amdgcn_readfirstlane(s_slow[k + 1]));
    compute_slow(j, k % kWaves);
    __syncthreads();  // the LDS buffers are rewritten by the next tile
  }

  // ---- cross-wave merge: common max M and total L per row, then the wave partials
  // are summed in LDS in MFMA register order, four output blocks per round
  const float l_row = l_run + swap_halves(l_run);
  __syncthreads();  // every wave is past its fast tiles (s_u is free)
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
  f32x4* buf = (f32x4*)s_u;  // [kWaves][4 blocks][4][64] f32x4
  f32x4* po = (f32x4*)(P.part_o + (int64_t)part * 32 * D);
  // only the item's rows move through LDS (lane l and thread t hold row l % 32 / t % 32)
  const bool my_row = (lane & 31) < nrows;
  // an item of one tile (a slow one, typically): wave 0 ran it and the other waves hold
  // O = 0, m = -inf, so only wave 0 writes and each thread reads wave 0's value alone
  const bool one = count == 1;
#pragma unroll
  for (int rb = 0; rb < C::MBLK / 4; ++rb) {
    if (my_row && (!one || wave == 0)) {
#pragma unroll
      for (int bb = 0; bb < 4; ++bb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16& Ob = O[4 * rb + bb];
          buf[((wave * 4 + bb) * 4 + q) * 64 + lane] =
              f32x4{Ob[4 * q] * fw, Ob[4 * q + 1] * fw, Ob[4 * q + 2] * fw, Ob[4 * q + 3] * fw};
        }
    }
    __syncthreads();
    if (my_row) {
      // f32x4 index e of the round is index 2 rb * kThreads + e of the partial
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = h * kThreads + tid;
        f32x4 acc = buf[e];
        if (!one) {
#pragma unroll
          for (int w = 1; w < kWaves; ++w) acc += buf[w * 2 * kThreads + e];
        }
        store_through(po, 2 * rb * kThreads + e, acc);
      }
    }
    __syncthreads();
  }
  if (tid < 32) {
    float lse = (L > 0.f && M != -INFINITY) ? (M + log2f(L)) * kLn2 : -INFINITY;
    if (M != M || L != L) lse = NAN;
    P.part_lse[(int64_t)part * 32 + tid] = lse;
  }
}

// FP32 LSE merge of a group's items (slab_attention.py:341-356 applied in
// sequence; empty parts contribute nothing).  One workgroup of W <= kMergeWaves
// waves per (group, 64-vector chunk of the register-order partial): lane l of every
// wave owns partial vector chunk * 64 + l, i.e. row l % 32, four d values.  Wave w
// merges items w, w + W, ... online (their partial vectors and LSEs loaded in
// batches of kBatch), then the W wave states (max, sum, vector) are combined in LDS
// by wave 0.  The host sizes W from the plan's items per group.
constexpr int kMergeWaves = 8;
constexpr int kBatch = 16;  // items per load round of a wave

template <int D>
__global__ __launch_bounds__(kMergeWaves * 64) void attn_merge_kernel(AttnParams P, StoreParams S) {
  using C = Cfg<D>;
  const oscar_attn_args_v1& A = P.a;
  // Workgroups past the groups (launched only for a deferred store, S.deferred) finish
  // that store: one wave per K / V vector quantizes the rotated vector the store's
  // rotation launch left in S.y and writes its slot bytes, FP32 window copy and owner
  // tag, as store_small_kernel's last slice workgroup does in the one-launch form.  It
  // runs beside the merge: nothing here reads the cache or the window.
  if ((int)blockIdx.x >= A.num_groups) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t hk = S.a.cache.num_kv_heads, nkv = S.a.num_tokens * hk;
    const int64_t v = ((int64_t)(blockIdx.x - A.num_groups) * gridDim.y + blockIdx.y) * (blockDim.x >> 6) + wave;
    if (!S.deferred || v >= 2 * nkv) return;
    const int kind = v < nkv ? KIND_K : KIND_V;
    const int64_t vw = kind == KIND_K ? v : v - nkv;
    const int64_t t = fdiv((uint32_t)vw, S.div_hk), h = vw - t * hk;
    const DestLoads dl = dest_loads(S, t);
    const f32x4 x4 = *(const f32x4*)(S.y + ((int64_t)kind * nkv + vw) * D + 4 * (lane < D / 4 ? lane : 0));
    const Dest dest = dest_finish(S, kind, t, dl);
    quant_vector<D>(S, kind, t, h, dest, x4);
    return;
  }
  // the group record carries everything the merge needs (no dependent loads)
  const int32_t* grp = A.groups + (int64_t)blockIdx.x * OSCAR_GROUP_INTS;
  const int kvh = grp[1], i0 = grp[2], ni = grp[3], a = grp[4], nq = grp[5];
  const int G = P.group;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int n = lane & 31, gg = lane >> 5;
  const int bq = blockIdx.y, b = bq >> 2, q = bq & 3;
  const int e = bq * 64 + lane;  // f32x4 index in the partial
  // a record that breaks oscar_attn_plan_v1's rules: rows outside the call are not
  // written at all; a bad item range turns the group's rows into NaN.  Branch-free up
  // to the stores (such a record reads no item and the NaN comes in with the result):
  // early exits here measured 0.25 us slower per merge at config 4a.
  const bool rows_bad = a < 0 || nq < 1 || nq * G > 32 || (int64_t)a + nq > A.num_tokens || kvh < 0 ||
                        kvh >= A.cache.num_kv_heads;
  const bool bad = i0 < 0 || ni < 0 || (int64_t)i0 + ni > A.num_items;
  const int nitems = (bad || rows_bad) ? 0 : ni;
  const bool row_ok = n < nq * G;
  const f32x4* po = (const f32x4*)P.part_o + (int64_t)(nitems ? i0 : 0) * C::NV + e;
  const float* pl = P.part_lse + (int64_t)(nitems ? i0 : 0) * 32 + n;
  float M = -INFINITY, L = 0.f;
  bool nan = bad;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int i = wave; i < nitems; i += W * kBatch) {
    float l[kBatch];
    f32x4 x[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int it = i + u * W;
      const bool in = it < nitems;
      l[u] = in ? pl[(int64_t)it * 32] : -INFINITY;
      x[u] = (in && row_ok) ? po[(int64_t)it * C::NV] : f32x4{0.f, 0.f, 0.f, 0.f};
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
  // combine the wave states: common max, rescaled sums (NaN in any wave wins)
  __shared__ f32x4 s_acc[kMergeWaves][64];
  __shared__ float s_m[kMergeWaves][64], s_l[kMergeWaves][64];
  __shared__ int s_nan[kMergeWaves][64];
  if (wave > 0) {
    s_acc[wave][lane] = acc;
    s_m[wave][lane] = M;
    s_l[wave][lane] = L;
    s_nan[wave][lane] = nan;
  }
  __syncthreads();
  if (wave > 0 || !row_ok) return;
  float Mt = M;
  for (int w = 1; w < W; ++w) {
    Mt = fmaxf(Mt, s_m[w][lane]);
    nan |= s_nan[w][lane] != 0;
  }
  if (Mt != -INFINITY) {
    const float f0 = (M == -INFINITY) ? 0.f : expf(M - Mt);
    acc *= f0;
    L *= f0;
    for (int w = 1; w < W; ++w) {
      const float mw = s_m[w][lane];
      const float f = (mw == -INFINITY) ? 0.f : expf(mw - Mt);
      if (f > 0.f) {
        acc += s_acc[w][lane] * f;
        L += s_l[w][lane] * f;
      }
    }
  }
  M = Mt;
  if (rows_bad) return;
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
int launch_decode(const AttnParams& p, hipStream_t s, const StoreParams& sp) {
  if (p.a.phases != 2) {
    if (p.a.q_dtype == OSCAR_F16)
      hipLaunchKernelGGL((attn_main_kernel<D, OSCAR_F16>), dim3(p.a.num_items), dim3(kThreads), 0, s, p);
    else
      hipLaunchKernelGGL((attn_main_kernel<D, OSCAR_BF16>), dim3(p.a.num_items), dim3(kThreads), 0, s, p);
    OSCAR_CHECK_LAUNCH("attn_main_kernel");
  }
  if (p.a.phases != 1) {
    // waves per merge workgroup: a power of two giving each wave one load round of
    // up to kBatch items of the largest group (8 x 24K MTP, 32 items per group: 2 waves
    // measured 0.2-0.3 us faster per step than 4, and 8 or 1 slower)
    const int per_group = p.a.max_group_items > 0 ? p.a.max_group_items : p.a.num_items;
    int waves = 1;
    while (waves < kMergeWaves && waves * kBatch < per_group) waves *= 2;
    // a deferred store's vectors: one per wave of the extra workgroups
    constexpr int64_t gy = Cfg<D>::NV / 64;
    const int64_t nvec = sp.deferred ? 2 * sp.a.num_tokens * sp.a.cache.num_kv_heads : 0;
    const int64_t extra = (nvec + gy * waves - 1) / (gy * waves);
    hipLaunchKernelGGL(attn_merge_kernel<D>, dim3((unsigned)(p.a.num_groups + extra), (unsigned)gy), dim3(waves * 64), 0,
                       s, p, sp);
    OSCAR_CHECK_LAUNCH("attn_merge_kernel");
  }
  return 0;
}

}  // namespace

}  // namespace oscar

using namespace oscar;

// ----------------------------------------------------------------- planning
namespace {

// Planning cost of a key tile in units of an INT2 history tile.  Tiles expected to
// hold staged tokens (the FP32 sink / recent window) or to need the slow path for
// another reason (current chunk, causal boundary, ragged end) move up to 64 KB of
// FP32 rows and run one at a time through the whole workgroup, against the 8 KB of
// code lines of a history tile that the eight waves stream concurrently.  16 was
// the measured ratio on MI355X when slow tiles moved their rows by LDS DMA one tile
// at a time (8 x 24K MTP and 64 mixed-length cache-only decodes both ended fastest
// with 12-16); with the rows loaded one tile ahead, 6-16 all measure the same.
constexpr int64_t kSlowCost = 16;
constexpr int64_t kMaxGroupItems = kMergeWaves * kBatch;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The key tiles of a (request, kv head) group as three ranges: head [0, he) (the
// expected sink window), body [he, ts) (INT2 history) and tail [ts, n) (the
// expected recent window and the slow-path tiles at the end).
struct PlanGroup {
  int req, kvh, n, he, ts;
  int qa, nq, seq, off;  // the (sub-)request: first query token, queries, visible keys, offset in the chunk
  int first_slot;
  int64_t kh, kb, kt;  // items of head, body, tail (split), or kb items over all tiles
  bool split;
};

// items of a range of nr tiles of cost c each when no item may cost more than C
int64_t range_items(int64_t nr, int64_t c, int64_t C, int64_t max_tiles) {
  if (nr <= 0) return 0;
  int64_t cap = C / c;
  if (cap < 1) cap = 1;
  if (cap > max_tiles) cap = max_tiles;
  return ceil_div(nr, cap);
}

// items when the group's tiles are dealt round-robin as one range: item i of k
// takes tiles i, i + k, ..., at most ceil(n / k) of them and at most
// ceil(nh / k) + ceil(nt / k) expensive ones (the head and tail are contiguous)
int64_t merged_items(const PlanGroup& G, int64_t C, int64_t max_tiles) {
  const int64_t n = G.n, nh = G.he, nt = G.n - G.ts;
  auto cost = [&](int64_t k) { return ceil_div(n, k) + (kSlowCost - 1) * (ceil_div(nh, k) + ceil_div(nt, k)); };
  int64_t lo = ceil_div(n, max_tiles), hi = n;
  if (lo < 1) lo = 1;
  if (hi < lo) hi = lo;
  if (cost(hi) > C) return hi;
  while (lo < hi) {
    const int64_t mid = (lo + hi) / 2;
    if (cost(mid) <= C) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// items of group G under the bound C: the cheaper of the split and merged layouts
// (split on a tie, which keeps the expensive tiles out of the history items);
// commit = record the choice in G
int64_t group_items(PlanGroup& G, int64_t C, int64_t max_tiles, bool commit) {
  if (G.n == 0) {
    if (commit) { G.split = false; G.kb = 1; G.kh = G.kt = 0; }
    return 1;
  }
  const int64_t kh = range_items(G.he, kSlowCost, C, max_tiles);
  const int64_t kb = range_items(G.ts - G.he, 1, C, max_tiles);
  const int64_t kt = range_items(G.n - G.ts, kSlowCost, C, max_tiles);
  const int64_t merged = merged_items(G, C, max_tiles);
  const bool split = kh + kb + kt <= merged;
  if (commit) {
    G.split = split;
    if (split) { G.kh = kh; G.kb = kb; G.kt = kt; }
    else { G.kh = G.kt = 0; G.kb = merged; }
  }
  return split ? kh + kb + kt : merged;
}

}  // namespace

extern "C" int oscar_attn_plan_v1(const int32_t* qsl, const int32_t* seqs, int32_t num_reqs,
                                  int32_t has_new, int32_t num_kv_heads, int32_t group,
                                  int32_t head_dim, int32_t chunk_tokens, int32_t target_items,
                                  int32_t sink_tokens, int32_t recent_tokens, int32_t* items,
                                  int32_t max_items, int32_t* groups, int32_t max_groups,
                                  oscar_plan_v1* plan) {
  if (!qsl || !seqs || !plan || num_reqs < 0 || num_kv_heads < 1 || num_kv_heads > 0xffff || group < 1 ||
      sink_tokens < 0 || recent_tokens < 0)
    return fail(-22, "oscar_attn_plan_v1: invalid arguments");
  if (head_dim != 128 && head_dim != 256)
    return fail(-22, "oscar_attn_plan_v1: head_dim %d unsupported (128/256)", head_dim);
  if (chunk_tokens < kTile) chunk_tokens = kTile;
  if (chunk_tokens > kMaxItemTokens) chunk_tokens = kMaxItemTokens;
  if (target_items < 1) target_items = 1;
  // Per group the tiles are cut into head / body / tail (PlanGroup) from the window
  // hint, and each range is dealt round-robin to its own items (item i of k: tiles
  // first + i, first + i + k, ...), or, where that takes fewer items, the whole group
  // is dealt as one range.  The bound C on an item's cost (history tiles + kSlowCost
  // per expected slow tile) is the smallest that keeps the item count within
  // target_items (at least one item per group; at most chunk_tokens keys per item).
  // A request with more than 32 rows per KV head is planned as sub-requests of
  // sub = 32 / group query tokens each (one 32-row MFMA tile): sub-request [a, b) of a
  // request of nq queries and length seq sees seq - nq + b keys and keeps the
  // request's causality (its query i sees keys [0, seq - nq + a + i + 1)); with a
  // current chunk, keys from seq - nq on are the chunk's, which the item record
  // carries as the sub-request's offset a in the chunk.
  if (group > 32) return fail(-22, "oscar_attn_plan_v1: %d query heads per KV head > 32", group);
  const int sub = 32 / group;
  int ngroups = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int nq = qsl[r + 1] - qsl[r];
    if (nq <= 0) continue;
    if (seqs[r] < 0 || (has_new && seqs[r] < nq))
      return fail(-22, "oscar_attn_plan_v1: sequence length must cover its query chunk");
    if (has_new && nq > (1 << 19)) return fail(-22, "oscar_attn_plan_v1: query chunk of request %d too long", r);
    ngroups += (int)ceil_div(nq, sub) * num_kv_heads;
    if (ngroups > (1 << 24)) return fail(-22, "oscar_attn_plan_v1: too many request x kv-head groups");
  }
  std::vector<PlanGroup> gl;
  gl.reserve((size_t)ngroups);
  for (int r = 0; r < num_reqs; ++r) {
    const int nq_all = qsl[r + 1] - qsl[r];
    for (int a = 0; a < nq_all; a += sub) {
      const int b = a + sub < nq_all ? a + sub : nq_all;
      const int nq = b - a;
      // (cache-only requests may be shorter than their queries: a sub-request that sees
      // no key keeps 0 keys, which leaves its rows empty as the request's own limit does)
      const int seq = seqs[r] - (nq_all - b) > 0 ? seqs[r] - (nq_all - b) : 0;
      const int off = has_new ? a : 0;
      const int hist = has_new ? seq - nq - off : seq;
      const int n = (int)ceil_div(seq, kTile);
      // the slow path takes every tile that reaches the first masked or current key
      int fe = hist < seq - nq + 1 ? hist : seq - nq + 1;
      if (fe < 0) fe = 0;
      int ts = fe / kTile;
      if (recent_tokens > 0) {
        const int w0 = seq - recent_tokens > 0 ? seq - recent_tokens : 0;
        if (w0 / kTile < ts) ts = w0 / kTile;
      }
      if (ts > n) ts = n;
      int he = 0;
      if (sink_tokens > 0) he = (int)ceil_div(sink_tokens < hist ? sink_tokens : hist, kTile);
      if (he >= ts) he = ts = 0;  // the expected window covers the group
      for (int h = 0; h < num_kv_heads; ++h)
        gl.push_back({r, h, n, he, ts, qsl[r] + a, nq, seq, off, 0, 0, 0, 0, false});
    }
  }
  const int64_t max_tiles = chunk_tokens / kTile;
  auto items_for = [&](int64_t C) {
    int64_t total = 0;
    for (PlanGroup& G : gl) total += group_items(G, C, max_tiles, false);
    return total;
  };
  int64_t lo = 1, hi = kSlowCost * max_tiles;
  while (lo < hi) {
    const int64_t mid = (lo + hi) / 2;
    if (items_for(mid) <= target_items) hi = mid;
    else lo = mid + 1;
  }
  // and no group of more items than one load round of the merge takes
  // (kMergeWaves x kBatch): one 24K request measured 35.4 us per step at 199 items,
  // 32.8 us at 118, with attn_main the same
  auto group_max = [&](int64_t C) {
    int64_t mx = 0;
    for (PlanGroup& G : gl) {
      const int64_t k = group_items(G, C, max_tiles, false);
      if (k > mx) mx = k;
    }
    return mx;
  };
  if (group_max(lo) > kMaxGroupItems) {
    int64_t glo = lo, ghi = kSlowCost * max_tiles;
    while (glo < ghi) {
      const int64_t mid = (glo + ghi) / 2;
      if (group_max(mid) <= kMaxGroupItems) ghi = mid;
      else glo = mid + 1;
    }
    lo = glo;
  }
  for (PlanGroup& G : gl) group_items(G, lo, max_tiles, true);
  int64_t nitems = 0, max_k = 0;
  for (PlanGroup& G : gl) {
    const int64_t k = G.split ? G.kh + G.kb + G.kt : G.kb;
    G.first_slot = (int)nitems;
    nitems += k;
    if (k > max_k) max_k = k;
    if (nitems > (1 << 26)) return fail(-22, "oscar_attn_plan_v1: too many work items");
  }
  // the item record keeps the tile stride (<= items of a group) in 12 bits
  if (max_k > kMaxStride) return fail(-22, "oscar_attn_plan_v1: %lld items in one group > %d", (long long)max_k, kMaxStride);
  plan->num_items = (int32_t)nitems;
  plan->num_groups = ngroups;
  plan->partial_bytes = nitems * 32 * (head_dim + 1) * (int64_t)sizeof(float);
  plan->max_group_items = (int32_t)max_k;
  plan->reserved = 0;
  if (items == nullptr || groups == nullptr) return (int)nitems;  // size query
  if (nitems > max_items || ngroups > max_groups) return fail(-28, "oscar_attn_plan_v1: buffers too small");
  // item p of a group: tail items, then head, then body (split), or item p of the
  // round-robin over all tiles (merged); tiles first + stride * i, i < count
  auto group_item = [&](const PlanGroup& G, int64_t p, int& first, int& stride, int& count) {
    int64_t a = 0, b = G.n, k = G.kb;
    if (G.split) {
      if (p < G.kt) { a = G.ts; b = G.n; k = G.kt; }
      else if ((p -= G.kt) < G.kh) { a = 0; b = G.he; k = G.kh; }
      else { p -= G.kh; a = G.he; b = G.ts; k = G.kb; }
    }
    first = (int)(a + p);
    stride = (int)k;
    count = b - a > p ? (int)ceil_div(b - a - p, k) : 0;
    if (count == 0) {
      first = 0;
      stride = 1;
    }
  };
  // Launch order: items interleaved over the groups (item p of every group, then
  // p + 1, ...), so that all groups progress together when there are more items
  // than compute units.  The partial slots of a group stay contiguous for the merge.
  int64_t idx = 0;
  for (int64_t pos = 0; pos < max_k; ++pos)
    for (const PlanGroup& G : gl) {
      const int64_t k = G.split ? G.kh + G.kb + G.kt : G.kb;
      if (pos >= k) continue;
      int32_t* it = items + idx++ * OSCAR_WORK_INTS;
      int first, stride, count;
      group_item(G, pos, first, stride, count);
      it[0] = G.req;
      it[1] = G.kvh | (G.nq << 16);
      it[2] = first;
      it[3] = stride | (G.off << 12);
      it[4] = count;
      it[5] = G.first_slot + (int)pos;
      it[6] = G.qa;
      it[7] = G.seq;
    }
  for (int q = 0; q < ngroups; ++q) {
    const PlanGroup& G = gl[(size_t)q];
    int32_t* gr = groups + (int64_t)q * OSCAR_GROUP_INTS;
    gr[0] = G.req;
    gr[1] = G.kvh;
    gr[2] = G.first_slot;
    gr[3] = (int)(G.split ? G.kh + G.kb + G.kt : G.kb);
    gr[4] = G.qa;
    gr[5] = G.nq;
    gr[6] = gr[7] = 0;
  }
  return (int)nitems;
}

namespace {

// Argument checks of a non-empty plan that do not depend on where the item partials
// go; `name` prefixes the messages.
int check_args(const oscar_attn_args_v1& a, const char* name) {
  const int64_t D = a.cache.head_dim;
  if (D != 128 && D != 256) return fail(-22, "%s: head_dim %lld unsupported", name, (long long)D);
  if (!a.q || !a.items || !a.groups || !a.out_rot || !a.lse || !a.block_table || !a.query_start_loc ||
      !a.seq_lens)
    return fail(-22, "%s: missing pointer", name);
  if ((a.k_new == nullptr) != (a.v_new == nullptr))
    return fail(-22, "%s: both new K and V must be supplied together", name);
  // streaming_attention.py:48-50; the coverage of each history (:51-53) is checked by the
  // kernel, which holds the lengths
  if (a.block_table_rows < a.num_reqs || a.block_table_cols < 1 || a.block_table_stride < a.block_table_cols)
    return fail(-22, "%s: Missing request block-table rows", name);
  if (a.phases < 0 || a.phases > 2) return fail(-22, "%s: phases must be 0, 1 or 2", name);
  if (a.q_dtype != OSCAR_BF16 && a.q_dtype != OSCAR_F16)
    return fail(-22, "%s: q_dtype must be OSCAR_BF16 or OSCAR_F16", name);
  if (a.cache.num_kv_heads < 1 || a.num_q_heads % a.cache.num_kv_heads)
    return fail(-22, "%s: Hq must be a multiple of Hk", name);
  if ((a.cache.k_stride[2] & 15) || (a.cache.v_stride[2] & 15) || (a.cache.k_stride[1] & 15) ||
      (a.cache.v_stride[1] & 15) || (a.cache.k_stride[0] & 15) || (a.cache.v_stride[0] & 15) ||
      (((uintptr_t)a.cache.k) & 15) || (((uintptr_t)a.cache.v) & 15))
    return fail(-22, "%s: cache slots must be 16-byte aligned", name);
  // queries and the current chunk are read as 16-byte vectors
  if ((a.q_stride_token & 7) || (((uintptr_t)a.q) & 15) ||
      (a.k_new && ((a.kv_new_stride_token & 7) || (((uintptr_t)a.k_new) & 15) || (((uintptr_t)a.v_new) & 15))))
    return fail(-22, "%s: q / k_new / v_new rows must be 16-byte aligned", name);
  if (a.cache.block_size < kTile || a.cache.block_size % kTile || a.cache.block_size > (1 << 20))
    return fail(-22, "%s: block_size %lld must be a multiple of %d (<= 2^20)", name,
                (long long)a.cache.block_size, kTile);
  if (a.staging && (a.staging->rows < 1 || a.staging->rows * a.cache.block_size >= (1ll << 31) ||
                    (((uintptr_t)a.staging->stage_k) & 15) || (((uintptr_t)a.staging->stage_v) & 15)))
    return fail(-22, "%s: staging arena rows out of range or unaligned", name);
  if (a.max_group_items < 0 || a.max_group_items > a.num_items)
    return fail(-22, "%s: max_group_items out of range", name);
  return 0;
}

// The decode entry points after their own checks.  `partials` / `partial_bytes`: where
// the item partials go and how much room there is.  `store` (oscar_decode_write_v1): the
// store enqueued once the decode's arguments have passed, deferred (its quantization in
// the merge launch) when it is a small call.
int launch_checked(const oscar_attn_args_v1& a, const char* name, void* partials, int64_t partial_bytes,
                   hipStream_t s, const oscar_store_args_v1* store = nullptr) {
  const int64_t D = a.cache.head_dim;
  if (D != 128 && D != 256) return fail(-22, "%s: head_dim %lld unsupported", name, (long long)D);
  if (a.num_items <= 0 || a.num_groups <= 0) {
    StoreParams sp{};
    return store != nullptr ? store_launch(store, s, false, name, &sp) : 0;
  }
  if (const int rc = check_args(a, name)) return rc;
  if (!partials) return fail(-22, "%s: missing workspace", name);
  const int64_t need = (int64_t)a.num_items * 32 * (D + 1) * (int64_t)sizeof(float);
  if (partial_bytes < need)
    return fail(-22, "%s: workspace of %lld bytes < %lld for %d items", name, (long long)partial_bytes,
                (long long)need, a.num_items);
  AttnParams p{};
  p.a = a;
  p.has_stage = a.staging != nullptr;
  if (a.staging) p.st = *a.staging;
  p.group = (int)(a.num_q_heads / a.cache.num_kv_heads);
  p.part_o = (float*)partials;
  p.part_lse = p.part_o + (int64_t)a.num_items * 32 * D;
  StoreParams sp{};
  if (store != nullptr) {
    if (store->cache.head_dim != D)
      return fail(-22, "%s: the store's head_dim %lld differs from the decode's", name,
                  (long long)store->cache.head_dim);
    const int rc = store_launch(store, s, a.phases == 0, name, &sp);
    if (rc != 0) return rc;
  }
  return D == 256 ? launch_decode<256>(p, s, sp) : launch_decode<128>(p, s, sp);
}

// ---- the entry point that allocates nothing: item partials in a file-scope device
// array.  Each device holds its own copy at its own address; host code must use the
// address hipGetSymbolAddress returns for the device (the array's name is a host-side
// stand-in), looked up once per device on the first call there.
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[OSCAR_DECODE_STATIC_MAX_ITEMS * 32 * (256 + 1) * sizeof(float)];
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int static_partials(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(-5, "oscar_attn_decode_static_v1: no current device");
  if (s != nullptr) {
    int sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess)
      return fail(-22, "oscar_attn_decode_static_v1: cannot query the stream's device");
    if (sdev != dev)
      return fail(-22, "oscar_attn_decode_static_v1: the stream belongs to device %d, the current device is %d",
                  sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(-22, "oscar_attn_decode_static_v1: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(-5, "oscar_attn_decode_static_v1: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int oscar_attn_decode_v1(const oscar_attn_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_attn_decode_v1: null args");
  return launch_checked(*args, "oscar_attn_decode_v1", args->workspace, args->workspace_bytes,
                        (hipStream_t)stream);
}

extern "C" int oscar_decode_write_v1(const oscar_store_args_v1* store, const oscar_attn_args_v1* attn,
                                     void* stream) {
  if (!store || !attn) return fail(-22, "oscar_decode_write_v1: null args");
  return launch_checked(*attn, "oscar_decode_write_v1", attn->workspace, attn->workspace_bytes, (hipStream_t)stream,
                        store);
}

extern "C" int oscar_attn_decode_static_v1(const oscar_attn_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_attn_decode_static_v1: null args");
  if (args->num_items > OSCAR_DECODE_STATIC_MAX_ITEMS)
    return fail(-22, "oscar_attn_decode_static_v1: %d items exceed the static scratch (at most %d)",
                args->num_items, OSCAR_DECODE_STATIC_MAX_ITEMS);
  if (args->num_items <= 0 || args->num_groups <= 0) return 0;
  if (const int rc = check_args(*args, "oscar_attn_decode_static_v1")) return rc;
  void* partials = nullptr;
  const int rc = static_partials((hipStream_t)stream, &partials);
  if (rc != 0) return rc;
  return launch_checked(*args, "oscar_attn_decode_static_v1", partials, (int64_t)sizeof(scratch),
                        (hipStream_t)stream);
}
