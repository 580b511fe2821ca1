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
// per SIMD) per item; wave w takes tiles w, w+4, ...; the four wave partials are
// merged in LDS and the item partial (normalised O, natural-log LSE) goes to the
// workspace; attn_merge_kernel combines the items of each group (FP32 LSE merge,
// slab_attention.py:341-356) into out_rot / lse.
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
//    P' = p*s_V (fp16) and sum_t p*z_V accumulates on the VALU (affine folded).
//  * slow tiles (staged tokens, current chunk, causal boundary, ragged end) are
//    deferred; the PV accumulators are then converted to value units and the
//    tiles are evaluated from full values rounded as the reference does.
#include "common.h"

namespace oscar {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <int D>
struct Cfg {
  static constexpr int KSTEPS = D / 16;  // QK contraction steps
  static constexpr int KDW = D / 32;     // K code dwords per lane (its half of D)
  static constexpr int NB = D / 4;       // code bytes per token
  static constexpr int MBLK = D / 32;    // PV output blocks (32 d each)
};

struct AttnParams {
  oscar_attn_args_v1 a;
  oscar_staging_v1 st;
  int has_stage;
  int group;     // Hq / Hk
  float* part_o;   // [num_items][32][D]
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

__device__ __forceinline__ float round_hist(float x) {
  // reference history rounding: fp16 then bf16 (streaming_attention.py:124)
  float h = __half2float(__float2half_rn(x));
  return bf16_bits_to_f32(f32_to_bf16_bits(h));
}

// d index of element e (0..7) of QK K-step j for lane half g
template <int D>
__device__ __forceinline__ int qk_d(int j, int g, int e) {
  return g * (D / 2) + 16 * (j >> 1) + 4 * (j & 1) + (e >> 1) + 8 * (e & 1);
}
// PV output block mb, row m -> d, and the code position of the block
template <int D>
__device__ __forceinline__ int pv_d(int mb, int m) {
  return (D == 256) ? 128 * (mb >> 2) + 4 * m + (mb & 3) : 4 * m + mb;
}
__device__ __forceinline__ int pv_pos(int mb) { return 2 * (mb & 3); }

// token (0..31) of MFMA K-element e for lane half g in PV K-step s
__device__ __forceinline__ int pv_tok(int s, int g, int e) {
  return 16 * s + 4 * g + (e & 3) + 8 * (e >> 2);
}
// token of S^T output register r for lane half g
__device__ __forceinline__ int out_tok(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

template <int D>
struct Item {
  int req, kvh, kb, ke;
  int a, nq, seq, hist, nrows;
};

template <int D>
__global__ __launch_bounds__(kThreads, 1) void attn_main_kernel(AttnParams P) {
  using C = Cfg<D>;
  const oscar_attn_args_v1& A = P.a;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 31, g = lane >> 5;
  const int32_t* it = A.items + (int64_t)blockIdx.x * OSCAR_WORK_INTS;
  Item<D> I;
  I.req = it[0]; I.kvh = it[1]; I.kb = it[2]; I.ke = it[3];
  I.a = A.query_start_loc[I.req];
  I.nq = A.query_start_loc[I.req + 1] - I.a;
  I.seq = A.seq_lens[I.req];
  const bool has_new = A.k_new != nullptr;
  I.hist = has_new ? I.seq - I.nq : I.seq;
  const int G = P.group;
  I.nrows = I.nq * G;
  const int64_t bs = A.cache.block_size;
  const int64_t hk = A.cache.num_kv_heads;

  // LDS
  __shared__ int32_t s_table[256 + 2];                 // block ids of the item's pages
  __shared__ __attribute__((aligned(16))) uint8_t s_vcode[kWaves][kTile * C::NB];
  __shared__ __attribute__((aligned(16))) float s_cst[kWaves][4][kTile];
  __shared__ __attribute__((aligned(16))) float s_ml[kWaves][2][32];
  // union: slow-tile V values (fp16) / cross-wave merge buffers
  __shared__ __attribute__((aligned(16))) uint8_t s_big[2 * D * 33 * 4];
  uint16_t* s_slowv = (uint16_t*)s_big + wave * (kTile * D);   // [32 tokens][D] fp16

  // page ids of the history pages this item reads; ids outside the cache are
  // clamped (the host validates tables, this keeps a bad table from faulting)
  const int page0 = I.kb / bs;
  const int hist_end = I.ke < I.hist ? I.ke : I.hist;
  const int npages = hist_end > I.kb ? (hist_end - 1) / bs - page0 + 1 : 0;
  for (int i = tid; i < npages; i += kThreads) {
    int32_t b = A.block_table[(int64_t)I.req * A.block_table_stride + page0 + i];
    s_table[i] = (b < 0 || b >= A.cache.num_blocks) ? 0 : b;
  }

  // ---- queries: lane (row n = m, half g) holds q[n][g*D/2 .. +D/2)
  const int n = m;
  const bool row_ok = n < I.nrows;
  const int qtok = I.a + (row_ok ? n / G : 0);
  const int qhead = I.kvh * G + (row_ok ? n % G : 0);
  const uint16_t* qrow = (const uint16_t*)A.q + (int64_t)qtok * A.q_stride_token + (int64_t)qhead * D;
  // Q^T operand (bf16, exact), element e of K-step j holds d = qk_d(j, g, e)
  bf16x8 qb[C::KSTEPS];
#pragma unroll
  for (int j = 0; j < C::KSTEPS; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      qb[j][e] = __builtin_bit_cast(__bf16, (unsigned short)(row_ok ? qrow[qk_d<D>(j, g, e)] : 0));
  const float c_score = A.scale * kLog2e;  // scores in log2 units
  __syncthreads();

  // ---- running state (per lane row n): max m_run (log2 units), partial sum l, z
  float m_run = -INFINITY, l_run = 0.f, z_run = 0.f;
  f32x16 O[C::MBLK];
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = 0.f;

  const int ntiles = (I.ke - I.kb + kTile - 1) / kTile;
  const int min_limit = I.seq - I.nq + 1;  // first key masked for some row
  uint64_t slow_mask = 0;
  const uint8_t* kbase = A.cache.k;
  const uint8_t* vbase = A.cache.v;
  const int64_t* owner = P.st.owner;
  const int64_t st_rows = P.st.rows;

  // move O, l, z (relative to m_run) to a new running max; wave-uniform
  auto update_max = [&](float mx) {
    const float m_new = fmaxf(m_run, mx);
    if (__any(m_new > m_run)) {
      const float f = (m_new == m_run) ? 1.f : (m_run == -INFINITY ? 0.f : exp2f(m_run - m_new));
#pragma unroll
      for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[b][r] *= f;
      l_run *= f;
      z_run *= f;
    }
    m_run = m_new;
  };

  for (int tile = wave, ti = 0; tile < ntiles; tile += kWaves, ++ti) {
    const int t0 = I.kb + tile * kTile;
    const int p = t0 + m;                   // this lane's token (lanes m, m+32 share it)
    const bool in_range = p < I.ke;
    const bool is_hist = in_range && p < I.hist;
    int64_t blk = 0, off = 0;
    bool staged = false;
    if (is_hist) {
      blk = s_table[p / bs - page0];
      off = p % bs;
      if (P.has_stage) {
        int64_t o = owner[((blk % st_rows) * bs + off)];
        staged = (o == blk);
      }
    }
    const bool tile_fast = (t0 + kTile <= I.ke) && (t0 + kTile <= I.hist) &&
                           (t0 + kTile <= min_limit) && !__any(staged);
    if (!tile_fast) {
      slow_mask |= 1ull << ti;
      continue;
    }
    // ---- loads: K codes (this lane's half), meta, V codes (this lane's half)
    const uint8_t* kslot = kbase + blk * A.cache.k_stride[0] + off * A.cache.k_stride[1] + I.kvh * A.cache.k_stride[2];
    const uint8_t* vslot = vbase + blk * A.cache.v_stride[0] + off * A.cache.v_stride[1] + I.kvh * A.cache.v_stride[2];
    unsigned kc[C::KDW], vc[C::KDW];
#pragma unroll
    for (int i = 0; i < C::KDW; i += 4) {
      u32x4 x = *(const u32x4*)(kslot + 32 + g * (D / 8) + 4 * i);
      kc[i] = x[0]; kc[i + 1] = x[1]; kc[i + 2] = x[2]; kc[i + 3] = x[3];
      u32x4 y = *(const u32x4*)(vslot + g * (D / 8) + 4 * i);
      vc[i] = y[0]; vc[i + 1] = y[1]; vc[i + 2] = y[2]; vc[i + 3] = y[3];
    }
    const u32x2 meta = *(const u32x2*)kslot;
    // V codes to LDS, natural layout [token][NB]
#pragma unroll
    for (int i = 0; i < C::KDW; i += 4) {
      u32x4 y = {vc[i], vc[i + 1], vc[i + 2], vc[i + 3]};
      *(u32x4*)&s_vcode[wave][m * C::NB + g * (D / 8) + 4 * i] = y;
    }
    // per-token V constants for the probability side
    if (g == 0) {
      s_cst[wave][2][m] = f16_bits_to_f32(meta[1] & 0xffff);
      s_cst[wave][3][m] = f16_bits_to_f32(meta[1] >> 16);
    }
    // ---- K operand: the 4 possible history values of this token, rounded exactly as
    // the reference (bf16(fp16(code*scale + zero))), form a byte table that v_perm_b32
    // indexes with 2*code, 2*code+1 per bf16 element.
    unsigned lut_lo, lut_hi;
    {
      const float sk = f16_bits_to_f32(meta[0] & 0xffff), zk = f16_bits_to_f32(meta[0] >> 16);
      unsigned short v[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = f32_to_bf16_bits(round_hist(__fadd_rn(__fmul_rn((float)c, sk), zk)));
      lut_lo = (unsigned)v[0] | ((unsigned)v[1] << 16);
      lut_hi = (unsigned)v[2] | ((unsigned)v[3] << 16);
    }
    // ---- S^T = K Q^T; element pair k of code dword w holds codes k and k+8
    f32x16 S = {};
#pragma unroll
    for (int i = 0; i < C::KDW; ++i) {
      const unsigned w = kc[i];
      unsigned o[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const unsigned y = (w >> (2 * k)) & 0x00030003u;
        o[k] = __builtin_amdgcn_perm(lut_hi, lut_lo, y * 0x202u + 0x01000100u);
      }
      const u32x4 a0 = {o[0], o[1], o[2], o[3]};
      const u32x4 a1 = {o[4], o[5], o[6], o[7]};
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a0), qb[2 * i], S, 0, 0, 0);
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a1), qb[2 * i + 1], S, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float xs[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      xs[r] = S[r] * c_score;
      mx = fmaxf(mx, xs[r]);
    }
    mx = fmaxf(mx, swap_halves(mx));
    update_max(mx);
    // probabilities; P' = p * s_V feeds the MFMA, sum p*z_V the VALU
    u32x4 pb[2];
    float lsum = 0.f, zsum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x4 sv = *(const f32x4*)&s_cst[wave][2][8 * q4 + 4 * g];
      const f32x4 zv = *(const f32x4*)&s_cst[wave][3][8 * q4 + 4 * g];
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const int r0 = 4 * q4 + i;
        float p0 = exp2f(xs[r0] - m_run), p1 = exp2f(xs[r0 + 1] - m_run);
        lsum += p0 + p1;
        zsum = fmaf(p0, zv[i], fmaf(p1, zv[i + 1], zsum));
        auto h = __builtin_amdgcn_cvt_pkrtz(p0 * sv[i], p1 * sv[i + 1]);
        pb[r0 >> 3][(r0 & 7) >> 1] = __builtin_bit_cast(unsigned, h);
      }
    }
    l_run += lsum;
    z_run += zsum;
    // ---- O^T += V^T P'^T, V^T from LDS via transpose reads
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
        unsigned x0 = (unsigned)tr[0], x1 = (unsigned)tr[1];
        unsigned t0 = __builtin_amdgcn_perm(0u, x0, 0x0C010C00u);
        unsigned t1 = __builtin_amdgcn_perm(0u, x0, 0x0C030C02u);
        unsigned t2 = __builtin_amdgcn_perm(0u, x1, 0x0C010C00u);
        unsigned t3 = __builtin_amdgcn_perm(0u, x1, 0x0C030C02u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          unsigned msk = 0x00030003u << (2 * k);
          u32x4 av = {t0 & msk, t1 & msk, t2 & msk, t3 & msk};
          const int mb = (D == 256) ? 4 * cp + k : k;
          O[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(av), __builtin_bit_cast(f16x8, pb[s]),
                                                         O[mb], 0, 0, 0);
        }
      }
    }
  }

  // ---- convert fast-tile accumulators to uniform units: O *= 2^(24-2k), += z
  const float z_row = z_run + swap_halves(z_run);
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b) {
    const float f = ldexpf(1.f, 24 - pv_pos(b));
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = fmaf(O[b][r], f, z_row);
  }
  // z has been applied with the weight of both halves; keep l per lane (summed later)

  // ---- slow tiles: full values with the reference rounding
  if (slow_mask) {
    for (int ti = 0; ti < 64; ++ti) {
      if (!((slow_mask >> ti) & 1)) continue;
      const int tile = wave + ti * kWaves;
      const int t0 = I.kb + tile * kTile;
      const int p = t0 + m;
      const bool in_range = p < I.ke && p < I.seq;
      const bool is_hist = in_range && p < I.hist;
      const bool is_cur = in_range && !is_hist;
      int64_t blk = 0, off = 0;
      bool staged = false;
      if (is_hist) {
        blk = s_table[p / bs - page0];
        off = p % bs;
        if (P.has_stage) staged = owner[(blk % st_rows) * bs + off] == blk;
      }
      // this lane's token values for its half of D (K) and all of D split by halves (V)
      const uint8_t* kslot = kbase + blk * A.cache.k_stride[0] + off * A.cache.k_stride[1] + I.kvh * A.cache.k_stride[2];
      const uint8_t* vslot = vbase + blk * A.cache.v_stride[0] + off * A.cache.v_stride[1] + I.kvh * A.cache.v_stride[2];
      float sk = 0.f, zk = 0.f, svv = 0.f, zvv = 0.f;
      if (is_hist && !staged) {
        u32x2 meta = *(const u32x2*)kslot;
        sk = f16_bits_to_f32(meta[0] & 0xffff); zk = f16_bits_to_f32(meta[0] >> 16);
        svv = f16_bits_to_f32(meta[1] & 0xffff); zvv = f16_bits_to_f32(meta[1] >> 16);
      }
      const int64_t seat = (blk % (st_rows > 0 ? st_rows : 1)) * bs + off;
      auto kval = [&](int d) -> float {
        if (!in_range) return 0.f;
        if (is_cur) {
          const uint16_t* kn = (const uint16_t*)A.k_new +
                               (int64_t)(I.a + p - I.hist) * A.kv_new_stride_token + I.kvh * D;
          return bf16_bits_to_f32(kn[d]);
        }
        if (staged) return round_hist(P.st.stage_k[(seat * hk + I.kvh) * D + d]);
        unsigned c = (kslot[32 + d / 4] >> (2 * (d & 3))) & 3u;
        return round_hist(__fadd_rn(__fmul_rn((float)c, sk), zk));  // mul, then add
      };
      auto vval = [&](int d) -> float {
        if (!in_range) return 0.f;
        if (is_cur) {
          const uint16_t* vn = (const uint16_t*)A.v_new +
                               (int64_t)(I.a + p - I.hist) * A.kv_new_stride_token + I.kvh * D;
          return bf16_bits_to_f32(vn[d]);
        }
        if (staged) return round_hist(P.st.stage_v[(seat * hk + I.kvh) * D + d]);
        unsigned c = (vslot[d / 4] >> (2 * (d & 3))) & 3u;
        return round_hist(__fadd_rn(__fmul_rn((float)c, svv), zvv));
      };
      f32x16 S = {};
#pragma unroll
      for (int j = 0; j < C::KSTEPS; ++j) {
        bf16x8 ka;  // full values, already on the bf16 grid
#pragma unroll
        for (int e = 0; e < 8; ++e)
          ka[e] = __builtin_bit_cast(__bf16, f32_to_bf16_bits(kval(qk_d<D>(j, g, e))));
        S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qb[j], S, 0, 0, 0);
      }
      // V values of this token to LDS (fp16), this lane's half of D
      for (int d = g * (D / 2); d < (g + 1) * (D / 2); ++d)
        s_slowv[m * D + d] = __half_as_ushort(__float2half_rn(vval(d)));
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      // masked scores
      float xs[16];
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tp = t0 + out_tok(r, g);
        const int limit = I.seq - I.nq + (row_ok ? n / G : 0) + 1;
        const bool vis = row_ok && tp < I.ke && tp < I.seq && tp < limit;
        xs[r] = vis ? S[r] * c_score : -INFINITY;
        mx = fmaxf(mx, xs[r]);
      }
      mx = fmaxf(mx, swap_halves(mx));
      update_max(mx);
      u32x4 pb[2];
      float lsum = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int r0 = 8 * s + 2 * q, r1 = r0 + 1;
          float p0 = (xs[r0] == -INFINITY) ? 0.f : exp2f(xs[r0] - m_run);
          float p1 = (xs[r1] == -INFINITY) ? 0.f : exp2f(xs[r1] - m_run);
          lsum += p0 + p1;
          auto h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
          pb[s][q] = __builtin_bit_cast(unsigned, h);
        }
      l_run += lsum;
#pragma unroll
      for (int b = 0; b < C::MBLK; ++b) {
        const int d = pv_d<D>(b, m);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          f16x8 va;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            va[e] = __builtin_bit_cast(_Float16, s_slowv[pv_tok(s, g, e) * D + d]);
          O[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, __builtin_bit_cast(f16x8, pb[s]), O[b], 0, 0, 0);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---- per-wave row totals
  const float l_row = l_run + swap_halves(l_run);
  // ---- cross-wave merge in LDS (deterministic tree: w0+w2, w1+w3, then w0+w1)
  __syncthreads();
  if (g == 0) { s_ml[wave][0][m] = m_run; s_ml[wave][1][m] = l_row; }
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][0][n]);
  float L = 0.f;
  for (int w = 0; w < kWaves; ++w) {
    float mw = s_ml[w][0][n];
    if (mw != -INFINITY) L += s_ml[w][1][n] * exp2f(mw - M);
  }
  const float fw = (m_run == -INFINITY || !(L > 0.f)) ? 0.f : exp2f(m_run - M) / L;
#pragma unroll
  for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] *= fw;
  float* buf = (float*)s_big;  // [2][D][33]
  auto put = [&](int slot) {
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) buf[(slot * D + pv_d<D>(b, out_tok(r, g))) * 33 + n] = O[b][r];
  };
  auto add = [&](int slot) {
#pragma unroll
    for (int b = 0; b < C::MBLK; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) O[b][r] += buf[(slot * D + pv_d<D>(b, out_tok(r, g))) * 33 + n];
  };
  if (wave >= 2) put(wave - 2);
  __syncthreads();
  if (wave < 2) add(wave);
  __syncthreads();
  if (wave == 1) put(0);
  __syncthreads();
  if (wave == 0) {
    add(0);
    put(0);
  }
  __syncthreads();
  // item partial: normalised O [32][D] and lse [32]
  const int part = it[4];
  float* po = P.part_o + (int64_t)part * 32 * D;
  for (int e = tid; e < 32 * D; e += kThreads) {
    int nn = e / D, dd = e % D;
    po[e] = buf[dd * 33 + nn];
  }
  if (tid < 32) {
    float lse = (L > 0.f && M != -INFINITY) ? (M + log2f(L)) * kLn2 : -INFINITY;
    if (M != M || L != L) lse = NAN;
    P.part_lse[(int64_t)part * 32 + tid] = lse;
  }
}

// One workgroup of D threads per (group, row): FP32 LSE merge of the group's items
// (slab_attention.py:341-356 applied in sequence; empty parts contribute nothing).
template <int D>
__global__ __launch_bounds__(D) void attn_merge_kernel(AttnParams P) {
  const oscar_attn_args_v1& A = P.a;
  const int32_t* grp = A.groups + (int64_t)blockIdx.x * 4;
  const int req = grp[0], kvh = grp[1], i0 = grp[2], i1 = grp[2] + grp[3];
  const int row = blockIdx.y;
  const int a = A.query_start_loc[req];
  const int nq = A.query_start_loc[req + 1] - a;
  const int G = P.group;
  if (row >= nq * G) return;
  const int tok = a + row / G, head = kvh * G + row % G;
  const int d = threadIdx.x;
  float M = -INFINITY;
  bool nan = false;
  for (int i = i0; i < i1; ++i) {
    float l = P.part_lse[(int64_t)i * 32 + row];
    nan |= (l != l);
    M = fmaxf(M, l);
  }
  float out = 0.f, lse = -INFINITY;
  if (nan) {
    out = NAN; lse = NAN;
  } else if (M != -INFINITY) {
    float acc = 0.f, L = 0.f;
    for (int i = i0; i < i1; ++i) {
      float l = P.part_lse[(int64_t)i * 32 + row];
      if (l == -INFINITY) continue;
      float w = expf(l - M);
      L += w;
      acc = fmaf(w, P.part_o[((int64_t)i * 32 + row) * D + d], acc);
    }
    out = acc / L;
    lse = M + logf(L);
  }
  A.out_rot[((int64_t)tok * A.num_q_heads + head) * D + d] = out;
  if (d == 0) A.lse[(int64_t)tok * A.num_q_heads + head] = lse;
}

template <int D>
int launch_decode(const AttnParams& p, hipStream_t s) {
  if (p.a.phases != 2) {
    hipLaunchKernelGGL(attn_main_kernel<D>, dim3(p.a.num_items), dim3(kThreads), 0, s, p);
    OSCAR_CHECK_LAUNCH("attn_main_kernel");
  }
  if (p.a.phases != 1) {
    hipLaunchKernelGGL(attn_merge_kernel<D>, dim3(p.a.num_groups, 32), dim3(D), 0, s, p);
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
  if (!qsl || !seqs || !plan || num_reqs < 0 || num_kv_heads < 1 || group < 1)
    return fail(-22, "oscar_attn_plan_v1: invalid arguments");
  if (head_dim != 128 && head_dim != 256)
    return fail(-22, "oscar_attn_plan_v1: head_dim %d unsupported (128/256)", head_dim);
  if (chunk_tokens < kTile) chunk_tokens = kTile;
  if (chunk_tokens > 8192) chunk_tokens = 8192;
  if (target_items < 1) target_items = 1;
  // total visible keys over (request, kv head) groups with queries
  int64_t total = 0;
  int ngroups = 0;
  for (int r = 0; r < num_reqs; ++r) {
    int nq = qsl[r + 1] - qsl[r];
    if (nq <= 0) continue;
    if (nq * group > 32) return fail(-22, "oscar_attn_plan_v1: request %d has %d rows > 32", r, nq * group);
    if (seqs[r] < 0 || (has_new && seqs[r] < nq))
      return fail(-22, "oscar_attn_plan_v1: sequence length must cover its query chunk");
    total += (int64_t)seqs[r] * num_kv_heads;
    ngroups += num_kv_heads;
  }
  int64_t total_tiles = 0;
  for (int r = 0; r < num_reqs; ++r)
    if (qsl[r + 1] > qsl[r]) total_tiles += (int64_t)((seqs[r] + kTile - 1) / kTile) * num_kv_heads;
  (void)total;
  // per group: items of whole tiles, proportional to the group's share of all
  // tiles (target_items overall), at most chunk_tokens (<= 8192) tokens each
  struct Grp { int req, kvh, ntiles, nitems, first_slot; };
  Grp* gl = (Grp*)alloca(sizeof(Grp) * (ngroups > 0 ? ngroups : 1));
  int gi = 0, nitems = 0, max_per_group = 0;
  for (int r = 0; r < num_reqs; ++r) {
    int nq = qsl[r + 1] - qsl[r];
    if (nq <= 0) continue;
    for (int h = 0; h < num_kv_heads; ++h) {
      int ntiles = (seqs[r] + kTile - 1) / kTile;
      int k = total_tiles > 0 ? (int)(((int64_t)ntiles * target_items * 2 + total_tiles) / (2 * total_tiles)) : 1;
      if (k < 1) k = 1;
      const int max_tiles = chunk_tokens / kTile;
      if ((ntiles + k - 1) / k > max_tiles) k = (ntiles + max_tiles - 1) / max_tiles;
      if (k > ntiles && ntiles > 0) k = ntiles;
      gl[gi] = {r, h, ntiles, k, nitems};
      nitems += k;
      if (k > max_per_group) max_per_group = k;
      ++gi;
    }
  }
  plan->num_items = nitems;
  plan->num_groups = ngroups;
  plan->partial_bytes = (int64_t)nitems * 32 * (head_dim + 1) * (int64_t)sizeof(float);
  if (items == nullptr || groups == nullptr) return nitems;  // size query
  if (nitems > max_items || ngroups > max_groups) return fail(-28, "oscar_attn_plan_v1: buffers too small");
  // Launch order interleaves groups (index = position * ngroups + group, compacted)
  // so that workgroup i runs on XCD i % 8 and a group's items share one L2; the
  // partial slots of a group stay contiguous for the merge.
  int idx = 0;
  for (int pos = 0; pos < max_per_group; ++pos) {
    for (int q = 0; q < ngroups; ++q) {
      if (pos >= gl[q].nitems) continue;
      const int k = gl[q].nitems;
      const int tb = (int)((int64_t)gl[q].ntiles * pos / k);
      const int te = (int)((int64_t)gl[q].ntiles * (pos + 1) / k);
      int32_t* it = items + (int64_t)idx * OSCAR_WORK_INTS;
      const int seq = seqs[gl[q].req];
      it[0] = gl[q].req;
      it[1] = gl[q].kvh;
      it[2] = tb * kTile;
      it[3] = te * kTile < seq ? te * kTile : seq;
      it[4] = gl[q].first_slot + pos;
      it[5] = q;
      it[6] = it[7] = 0;
      ++idx;
    }
  }
  for (int q = 0; q < ngroups; ++q) {
    groups[q * 4 + 0] = gl[q].req;
    groups[q * 4 + 1] = gl[q].kvh;
    groups[q * 4 + 2] = gl[q].first_slot;
    groups[q * 4 + 3] = gl[q].nitems;
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
      (a.cache.v_stride[1] & 15) || (((uintptr_t)a.cache.k) & 15) || (((uintptr_t)a.cache.v) & 15))
    return fail(-22, "oscar_attn_decode_v1: cache slots must be 16-byte aligned");
  if (a.cache.block_size < 1 || 8192 / a.cache.block_size + 2 > 256)
    return fail(-22, "oscar_attn_decode_v1: block_size %lld too small for the page table stage",
                (long long)a.cache.block_size);
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
