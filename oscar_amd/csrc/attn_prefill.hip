// Causal GQA prefill over an optional INT2 history for gfx950 (MFMA bf16).
//
// Replaces oscar_ascend/kernels/prefill.py:69-72 / decode_kernel.py:70-117
// (fresh-only prefill: causal SDPA of the current chunk, original domain, bf16 out)
// and the long-continuation use of slab_attention.py:376-476 (history waves plus
// the causal current chunk, rotated domain, fp32 out + LSE).
//
// Query i (0-based in the chunk) sees keys [0, history + i + 1).
//
// Two launches when there is a history:
//   history_bf16_kernel  the history's K/V values with the reference rounding
//                        (q_dtype(fp16(code*scale + zero)), or the staged fp32 value
//                        when the seat's owner tag matches, prepare_kv.py:77) into a
//                        caller-provided bf16 workspace, once per call: every query
//                        tile of a long chunk reuses them;
//   prefill_kernel       flash attention over [workspace history | current chunk].
//                        A workgroup of four waves owns 128 query rows (tokens x heads
//                        of one KV head, GQA packed; Q^T operands in LDS).  Key tiles of
//                        32 are double-buffered in LDS: each thread prefetches its
//                        share of tile t+2 into registers while tile t is computed, so
//                        one barrier per tile separates the buffers.  Per wave:
//                        S^T = K Q^T (v_mfma_f32_32x32x16_bf16 / _f16), online softmax
//                        in fp32 (log2 domain) with a lazy reference max, O^T += V^T P^T
//                        on v_mfma_f32_32x32x16_f16 (P and V in fp16, see kVShift) with
//                        V^T read from LDS by ds_read_b64_tr_b16.
#include "common.h"

namespace oscar {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 256;
constexpr int kKeys = 32;
constexpr int kRows = 128;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazy = 8.f;  // max drift (log2 units) before O is rescaled
constexpr int kQK = 4;        // QK K-steps whose LDS operands are read together
// PV runs on v_mfma_f32_32x32x16_f16 with P and V in fp16 for both query dtypes.  bf16
// V values (8-bit significands) are held as fp16(v * 2^-kVShift): exact for |v| from
// 2^-6 up to 2^23 (below, within 2^-17 absolutely), and O is scaled back by 2^kVShift.
constexpr int kVShift = 8;
typedef short __attribute__((ext_vector_type(4))) i16x4;
typedef __bf16 __attribute__((ext_vector_type(2))) bf16x2;
typedef _Float16 __attribute__((ext_vector_type(2))) f16x2;
typedef float __attribute__((ext_vector_type(2))) f32x2;

// the reference history value q_dtype(fp16(x)) (prepare_kv.py:77) as 16-bit bits
template <int QT>
__device__ __forceinline__ unsigned hist_bits(float x) {
  const __half h = __float2half_rn(x);
  if constexpr (QT == OSCAR_F16) return __half_as_ushort(h);
  else return f32_to_bf16_bits(__half2float(h));
}
// 16-bit bits of x in the query dtype (RNE)
template <int QT>
__device__ __forceinline__ unsigned q_bits(float x) {
  if constexpr (QT == OSCAR_F16) return f32_to_f16_bits(x);
  else return f32_to_bf16_bits(x);
}
// the PV operand bits of a value v already in the query dtype: fp16 as it is; a bf16
// value scaled by 2^-kVShift into fp16 (exact, see kVShift)
template <int QT>
__device__ __forceinline__ unsigned pv_bits(float v) {
  if constexpr (QT == OSCAR_F16) return f32_to_f16_bits(v);
  else return f32_to_f16_bits(v * (1.f / (1 << kVShift)));
}
template <int QT> struct QVec { typedef bf16x8 type; typedef bf16x2 pair; typedef __bf16 elem; };
template <> struct QVec<OSCAR_F16> { typedef f16x8 type; typedef f16x2 pair; typedef _Float16 elem; };

// ---- balanced split of the key ranges (a workspace of oscar_prefill_workspace_bytes_v2)
// Query tile qt (kRows GQA rows) sees key tiles [0, kt(qt)), kt growing with qt under
// the causal mask.  One workgroup per tile leaves the chip unbalanced: the continuation
// of 15360 + 9256 tokens is 441 tiles of 481..771 key tiles on 256 CUs (1.7 rounds), a
// fresh 2048-token prefill 96 tiles (a third of the CUs).  The key range of a tile is
// instead cut into chunks of U key tiles (c U .. (c + 1) U), U about the work of half a
// CU, and every chunk is a workgroup ("unit"); a tile with more than one chunk writes
// normalised partials + log2 LSEs, and prefill_merge_kernel combines them (FP32 LSE
// merge).  Units are numbered chunk-major, heaviest tile first within a chunk index,
// so the large units are dispatched first: the tiles that have a chunk c are the
// suffix qt >= qmin[c] (kt is non-decreasing in qt), and unit u of chunk class c
// (base[c] <= u < base[c + 1]) is tile ntq - 1 - (u - base[c]).
constexpr int kMaxChunks = 32;
constexpr int64_t kMinChunkTiles = 16;  // 512 keys: shorter chunks cost more in merge than they balance
constexpr int64_t kSplitCUs = 256;      // MI355X compute units
constexpr int64_t kUnitsPerCU = 2;

struct PrefillParams {
  oscar_prefill_args_v1 a;
  oscar_staging_v1 st;
  int has_stage;
  int group;
  int qtok;            // query tokens per workgroup
  uint16_t* hist_k;    // [history][Hk][D] bf16 history values (workspace)
  uint16_t* hist_v;
  // the split plan (split == 0: one unit per query tile, the whole key range)
  int split;
  int chunks;          // chunks of the heaviest tile
  int U;               // key tiles per chunk
  int ntq;             // query tiles
  int qmin1;           // first tile with two chunks (the split tiles are qt >= qmin1)
  int base[kMaxChunks + 1];
  float* part_o;       // [slot][Hk][kRows][D] normalised partial O of the split tiles' chunks
  float* part_lse;     // [slot][Hk][kRows] log2-domain LSE of each partial
};

// key tiles seen by the last query of a tile ending at chunk token q1
__host__ __device__ inline int64_t tile_keys(int64_t hist, int64_t q1) { return (hist + q1 + kKeys - 1) / kKeys; }

struct SplitPlan {
  int chunks = 0, U = 0, ntq = 0, units = 0, qmin1 = 0;
  int base[kMaxChunks + 1] = {};
  int64_t slots = 0;   // partial slots per KV head
};

SplitPlan plan_split(int64_t hist, int64_t n, int64_t qtok, int64_t hk) {
  SplitPlan sp;
  if (n <= 0) return sp;
  const int64_t ntq = (n + qtok - 1) / qtok;
  auto kt = [&](int64_t qt) { return tile_keys(hist, (qt + 1) * qtok < n ? (qt + 1) * qtok : n); };
  int64_t work = 0;
  for (int64_t qt = 0; qt < ntq; ++qt) work += kt(qt);
  const int64_t kmax = kt(ntq - 1);
  int64_t U = (work * hk + kSplitCUs * kUnitsPerCU - 1) / (kSplitCUs * kUnitsPerCU);
  if (U < kMinChunkTiles) U = kMinChunkTiles;
  if ((kmax + U - 1) / U > kMaxChunks) U = (kmax + kMaxChunks - 1) / kMaxChunks;
  const int64_t chunks = (kmax + U - 1) / U;
  if (chunks < 2 || ntq > (1 << 24) || U > (1 << 24)) return sp;
  sp.chunks = (int)chunks;
  sp.U = (int)U;
  sp.ntq = (int)ntq;
  // qmin[c]: first tile with kt > c U (kt non-decreasing in qt)
  int64_t qt = 0, units = 0;
  for (int c = 0; c < sp.chunks; ++c) {
    while (qt < ntq && kt(qt) <= c * U) ++qt;
    if (c == 1) sp.qmin1 = (int)qt;
    sp.base[c] = (int)units;
    units += ntq - qt;
  }
  sp.base[sp.chunks] = (int)units;
  sp.units = (int)units;
  sp.slots = units - sp.qmin1;  // every unit but the single-chunk tiles' (class 0, qt < qmin1)
  return sp;
}

constexpr int64_t kWsAlign = 256;
int64_t hist_bytes(int64_t history, int64_t hk, int64_t D) {
  return history > 0 ? (2 * history * hk * D * (int64_t)sizeof(uint16_t) + kWsAlign - 1) / kWsAlign * kWsAlign : 0;
}
int64_t split_bytes(const SplitPlan& sp, int64_t hk, int64_t D) {
  return sp.chunks < 2 ? 0 : sp.slots * hk * kRows * (D + 1) * (int64_t)sizeof(float);
}

// one wave per (history token, kv head): lane l holds elements E*l .. E*l+E-1
template <int D, int QT>
__global__ __launch_bounds__(256) void history_bf16_kernel(PrefillParams P) {
  constexpr int E = D / 64;
  const oscar_prefill_args_v1& A = P.a;
  const int64_t hk = A.num_kv_heads;
  const int64_t vec = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (vec >= A.history * hk) return;
  const int lane = threadIdx.x & 63;
  const int64_t p = vec / hk, h = vec % hk;
  const int64_t bs = A.cache.block_size;
  int64_t blk = A.block_table_row[p / bs];
  if (blk < 0 || blk >= A.cache.num_blocks) blk = 0;  // host validates; never fault
  const int64_t off = p % bs;
  int64_t seat = 0;
  bool staged = false;
  if (P.has_stage) {
    seat = (blk % P.st.rows) * bs + off;
    staged = P.st.owner[seat] == blk;
  }
  float kv[E], vv[E];
  if (staged) {
    const float* sk = P.st.stage_k + (seat * hk + h) * D + E * lane;
    const float* sv = P.st.stage_v + (seat * hk + h) * D + E * lane;
#pragma unroll
    for (int i = 0; i < E; ++i) { kv[i] = sk[i]; vv[i] = sv[i]; }
  } else {
    const uint8_t* ks = A.cache.k + blk * A.cache.k_stride[0] + off * A.cache.k_stride[1] + h * A.cache.k_stride[2];
    const uint8_t* vs = A.cache.v + blk * A.cache.v_stride[0] + off * A.cache.v_stride[1] + h * A.cache.v_stride[2];
    const unsigned m0 = *(const unsigned*)ks, m1 = *(const unsigned*)(ks + 4);
    const float sk = f16_bits_to_f32(m0 & 0xffff), zk = f16_bits_to_f32(m0 >> 16);
    const float sv = f16_bits_to_f32(m1 & 0xffff), zv = f16_bits_to_f32(m1 >> 16);
    const int e0 = E * lane;  // element e sits in byte e / 4, bits 2 (e % 4)
    const unsigned kb = ks[32 + e0 / 4], vb = vs[e0 / 4];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int sh = 2 * ((e0 + i) & 3);
      kv[i] = __fadd_rn(__fmul_rn((float)((kb >> sh) & 3u), sk), zk);
      vv[i] = __fadd_rn(__fmul_rn((float)((vb >> sh) & 3u), sv), zv);
    }
  }
  unsigned kw[E / 2], vw[E / 2];
#pragma unroll
  for (int i = 0; i < E / 2; ++i) {
    kw[i] = hist_bits<QT>(kv[2 * i]) | (hist_bits<QT>(kv[2 * i + 1]) << 16);
    // V: the reference's history value in the query dtype, then the PV operand bits
    const unsigned v0 = hist_bits<QT>(vv[2 * i]), v1 = hist_bits<QT>(vv[2 * i + 1]);
    auto as_float = [](unsigned b) {
      return QT == OSCAR_F16 ? f16_bits_to_f32((unsigned short)b) : bf16_bits_to_f32((unsigned short)b);
    };
    vw[i] = pv_bits<QT>(as_float(v0)) | (pv_bits<QT>(as_float(v1)) << 16);
  }
  uint16_t* dk = P.hist_k + vec * D + E * lane;
  uint16_t* dv = P.hist_v + vec * D + E * lane;
  if constexpr (E == 4) {
    *(u32x2*)dk = u32x2{kw[0], kw[1]};
    *(u32x2*)dv = u32x2{vw[0], vw[1]};
  } else {
    *(unsigned*)dk = kw[0];
    *(unsigned*)dv = vw[0];
  }
}

template <int D, int QT>
__global__ __launch_bounds__(kThreads, 1) void prefill_kernel(PrefillParams P) {
  using QV = typename QVec<QT>::type;    // one MFMA operand in the query dtype
  const oscar_prefill_args_v1& A = P.a;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 31, g = lane >> 5;
  const int G = P.group;
  const int ntiles_q = (int)((A.num_tokens + P.qtok - 1) / P.qtok);
  const int kvh = blockIdx.y;
  const int64_t hist = A.history;
  const int64_t hk = A.num_kv_heads;
  // this workgroup's unit: query tile qt over key tiles [kb, ke); slot >= 0: the tile
  // is split and this unit writes a partial
  int qt, kb = 0, slot = -1;
  if (P.split) {
    const int u = blockIdx.x;
    int c = 0;
#pragma unroll
    for (int cc = 1; cc < kMaxChunks; ++cc)
      if (cc < P.chunks && u >= P.base[cc]) c = cc;
    const int idx = u - P.base[c];
    qt = ntiles_q - 1 - idx;  // heaviest (latest) query tiles first within a chunk class
    kb = c * P.U;
    if (qt >= P.qmin1) slot = c == 0 ? idx : u - P.qmin1;
  } else {
    qt = ntiles_q - 1 - (int)blockIdx.x;  // heaviest (latest) query tiles first
  }
  const int64_t q0 = (int64_t)qt * P.qtok;
  const int64_t q1 = (q0 + P.qtok < A.num_tokens) ? q0 + P.qtok : A.num_tokens;
  const int64_t nkeys = hist + q1;  // keys visible to the last query of the tile

  // double-buffered key tiles.  K rows are padded by 16 bytes (row-per-lane 16-byte
  // reads of 8 consecutive keys cover all banks), V rows by 32 bytes (the transpose
  // reads of 4 consecutive keys x 32 bytes cover all banks)
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kKeys][D + 8];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[2][kKeys][D + 16];

  // fill mapping: pass i, thread -> key i * KPP + tid / CPR, 16-byte column tid % CPR,
  // so that a wave reads (and stores to LDS) whole contiguous key rows
  constexpr int CPR = D / 8;              // 16-byte columns per key row
  constexpr int KPP = kThreads / CPR;     // keys per pass
  constexpr int NPASS = kKeys / KPP;
  const int fkey = tid / CPR, fcol = tid % CPR;
  u32x4 kr[NPASS], vr[NPASS];
  bool vcur[NPASS];  // the V row is a current-chunk row (query dtype, not PV format)
  // branch-free, 32-bit element offsets (the host checks they fit): keys past the
  // chunk read current-chunk row 0, finite data whose scores the causal mask removes
  const uint16_t* hk_base = P.hist_k + kvh * D + 8 * fcol;
  const uint16_t* hv_base = P.hist_v + kvh * D + 8 * fcol;
  const uint16_t* ck_base = (const uint16_t*)A.k + kvh * D + 8 * fcol;
  const uint16_t* cv_base = (const uint16_t*)A.v + kvh * D + 8 * fcol;
  const int hrow = (int)(hk * D), crow = (int)A.kv_stride_token;
  const int ihist = (int)hist, ikeys = (int)nkeys;
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
      const int p = kt * kKeys + i * KPP + fkey;
      const bool in_hist = p < ihist;
      const int ci = (in_hist || p >= ikeys) ? 0 : p - ihist;  // current-chunk index
      const uint16_t* ks = in_hist ? hk_base + (unsigned)(p * hrow) : ck_base + (unsigned)(ci * crow);
      const uint16_t* vs = in_hist ? hv_base + (unsigned)(p * hrow) : cv_base + (unsigned)(ci * crow);
      kr[i] = *(const u32x4*)ks;
      vr[i] = *(const u32x4*)vs;
      vcur[i] = !in_hist;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
      *(u32x4*)&s_k[buf][i * KPP + fkey][8 * fcol] = kr[i];
      u32x4 w = vr[i];
      if constexpr (QT == OSCAR_BF16) {
        if (vcur[i]) {  // bf16 current-chunk values to the PV format
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = pv_bits<QT>(__uint_as_float(vr[i][e] << 16)) | (pv_bits<QT>(__uint_as_float(vr[i][e] & 0xffff0000u)) << 16);
        }
      }
      *(u32x4*)&s_v[buf][i * KPP + fkey][8 * fcol] = w;
    }
  };

  const int kt_all = (int)tile_keys(hist, q1);
  const int ke = (P.split && kb + P.U < kt_all) ? kb + P.U : kt_all;  // kb < kt_all (plan)
  fetch(kb);

  // this lane's row
  const int n = wave * 32 + m;
  const int64_t qi = q0 + n / G;
  const bool row_ok = (n < P.qtok * G) && (qi < q1);
  const int head = kvh * G + n % G;
  const uint16_t* qrow = (const uint16_t*)A.q + (row_ok ? qi : 0) * A.q_stride_token + (int64_t)head * D;
  // the wave's Q^T operands (K-step j) in registers for the whole key range: each
  // tile's QK then reads only K from LDS
  QV qreg[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j)
    qreg[j] = __builtin_bit_cast(QV, row_ok ? *(const u32x4*)(qrow + 16 * j + 8 * g) : u32x4{0u, 0u, 0u, 0u});
  const float c = A.scale * kLog2e;
  const int64_t limit = hist + qi + 1;  // keys [0, limit) visible to this row

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 O[D / 32];
#pragma unroll
  for (int b = 0; b < D / 32; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = 0.f;

  stash(kb & 1);
  if (kb + 1 < ke) fetch(kb + 1);
  __syncthreads();
  // The tile loop does no VALU work on O (kept in AGPRs by the MFMAs): a tile whose
  // row max drifts more than kLazy above the reference leaves the loop, O and l are
  // rescaled once, and the loop resumes at that tile (its QK is recomputed).
  int kt = kb;
  float m_move = -INFINITY;  // per row: the max that forced the exit
  while (true) {
    for (; kt < ke; ++kt) {
      const int buf = kt & 1;
      const int64_t k0 = (int64_t)kt * kKeys;
      // ---- S^T = K Q^T; the operands of kQK K-steps are read from LDS together so
      // that one LDS latency covers kQK MFMAs
      f32x16 S = {};
#pragma unroll
      for (int j0 = 0; j0 < D / 16; j0 += kQK) {
        QV ka[kQK], qa[kQK];
#pragma unroll
        for (int j = 0; j < kQK; ++j) {
          ka[j] = *(const QV*)&s_k[buf][m][16 * (j0 + j) + 8 * g];
          qa[j] = qreg[j0 + j];
        }
#pragma unroll
        for (int j = 0; j < kQK; ++j) {
          if constexpr (QT == OSCAR_F16) S = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[j], qa[j], S, 0, 0, 0);
          else S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[j], qa[j], S, 0, 0, 0);
        }
        // keep the group's LDS reads ahead of its MFMAs (one latency per group)
        __builtin_amdgcn_sched_group_barrier(0x100, kQK, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kQK, 0);
      }
      const bool full = (k0 + kKeys <= hist + q0 + 1);  // visible to every row of the tile
      // masked keys get -inf scores (boundary tiles only).  Padding rows have zero
      // queries and are never written, so they need no mask.
      if (!full) {
        const int lim = (int)(limit - k0);  // keys of the tile visible to this row
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int pk = 8 * (r >> 2) + 4 * g + (r & 3);
          S[r] = pk >= lim ? -INFINITY : S[r];
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S[r]);
      {
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;  // c > 0
      }
      // a row's first visible key sets its reference (O and l are still zero there)
      if (m_run == -INFINITY) m_run = mx;
      if (__any(mx > m_run + kLazy)) {
        m_move = mx;
        break;
      }
      // p = 2^(S c - m) (exp2 of -inf is 0); rows with no key yet keep m = -inf and p = 0
      const float nm = (m_run == -INFINITY) ? 0.f : -m_run;
      // P in fp16 (p <= 2^kLazy; relative error 2^-12 per element)
      f16x8 pb[2];
      float lsum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(S[r], c, nm));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(S[r + 1], c, nm));
        lsum += p0 + p1;
        const f16x2 h = __builtin_convertvector(f32x2{p0, p1}, f16x2);
        pb[r >> 3][r & 7] = h[0];
        pb[r >> 3][(r & 7) + 1] = h[1];
      }
      l_run += lsum;
      // ---- O^T += V^T P^T; the V^T operands of two output blocks (8 transpose reads)
      // are read together
      const int G16 = lane >> 4, i16 = lane & 15;
#pragma unroll
      for (int b0 = 0; b0 < D / 32; b0 += 2) {
        f16x8 va[2][2];
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int key = 16 * s + 4 * (G16 >> 1) + 8 * h + (i16 >> 2);
              const uint16_t* addr = &s_v[buf][key][32 * (b0 + bb) + 16 * (G16 & 1) + 4 * (i16 & 3)];
              auto t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(addr));
#pragma unroll
              for (int e = 0; e < 4; ++e) va[bb][s][4 * h + e] = __builtin_bit_cast(_Float16, (unsigned short)t[e]);
            }
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int s = 0; s < 2; ++s)
            O[b0 + bb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[bb][s], pb[s], O[b0 + bb], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
      }
      // the prefetched tile kt+1 goes to the other buffer (last read before the previous
      // barrier), then tile kt+2 is prefetched; one barrier per tile
      if (kt + 1 < ke) {
        stash(buf ^ 1);
        if (kt + 2 < ke) fetch(kt + 2);
      }
      __syncthreads();
    }
    if (kt >= ke) break;
    // rare: rescale to the new reference and redo tile kt (its buffers are intact)
    const bool move = m_move > m_run + kLazy;
    const float f = move ? exp2f(m_run - m_move) : 1.f;
#pragma unroll
    for (int b = 0; b < D / 32; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) O[b][r] *= f;
    l_run *= f;
    if (move) m_run = m_move;
  }
  // ---- finalize: row n = lane's row; O^T block b register r holds d = 32b + out_row(r, g)
  float l_tot;
  {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_tot = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (!row_ok) return;
  // O back from the PV scale of bf16 V values (a power of two: exact)
  const float inv = (l_tot > 0.f) ? (QT == OSCAR_F16 ? 1.f : (float)(1 << kVShift)) / l_tot : 0.f;
  if (slot >= 0) {
    // a chunk of a split tile: normalised O and its log2-domain LSE (-inf: no key of
    // the chunk visible to the row) for prefill_merge_kernel
    const int64_t prow = ((int64_t)slot * hk + kvh) * kRows + n;
    float* po = P.part_o + prow * D;
#pragma unroll
    for (int b = 0; b < D / 32; ++b)
#pragma unroll
      for (int r = 0; r < 16; r += 4)
        *(f32x4*)(po + 32 * b + 8 * (r >> 2) + 4 * g) =
            f32x4{O[b][r] * inv, O[b][r + 1] * inv, O[b][r + 2] * inv, O[b][r + 3] * inv};
    if (g == 0) P.part_lse[prow] = (l_tot > 0.f) ? m_run + log2f(l_tot) : -INFINITY;
    return;
  }
  const int64_t obase = qi * A.out_stride_token + (int64_t)head * D;
#pragma unroll
  for (int b = 0; b < D / 32; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * b + 8 * (r >> 2) + 4 * g + (r & 3);
      const float v = O[b][r] * inv;
      if (hist == 0) ((uint16_t*)A.out)[obase + d] = (uint16_t)q_bits<QT>(v);
      else ((float*)A.out)[obase + d] = v;
    }
  if (A.lse != nullptr && g == 0)
    A.lse[qi * A.num_q_heads + head] = (l_tot > 0.f) ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
}

// FP32 LSE merge of a split tile's chunk partials (slab_attention.py:341-356 applied
// over the chunks): thread (row, 4 d values), D / 4 threads per row.  Writes what the
// unsplit kernel writes for the row: the output (query dtype when there is no history,
// else fp32 rotated) and the LSE.
template <int D, int QT>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams P) {
  constexpr int TPR = D / 4, RPW = 256 / TPR, WPT = kRows / RPW;
  const oscar_prefill_args_v1& A = P.a;
  const int s = blockIdx.x / WPT;  // split tile, heaviest first (its class-0 slot)
  const int n = (blockIdx.x % WPT) * RPW + threadIdx.x / TPR;
  const int dq = threadIdx.x % TPR;
  const int kvh = blockIdx.y;
  const int64_t hk = A.num_kv_heads;
  const int G = P.group;
  const int qt = P.ntq - 1 - s;
  const int64_t q0 = (int64_t)qt * P.qtok;
  const int64_t q1 = (q0 + P.qtok < A.num_tokens) ? q0 + P.qtok : A.num_tokens;
  const int64_t qi = q0 + n / G;
  if (n >= P.qtok * G || qi >= q1) return;
  const int nch = (int)((tile_keys(A.history, q1) + P.U - 1) / P.U);
  auto prow = [&](int c) {
    const int64_t slot = c == 0 ? s : P.base[c] + s - P.qmin1;
    return (slot * hk + kvh) * kRows + n;
  };
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c)
    if (c < nch) M = fmaxf(M, P.part_lse[prow(c)]);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      if (c < nch) {
        const int64_t r = prow(c);
        const float lc = P.part_lse[r];
        if (lc != -INFINITY) {
          const float w = exp2f(lc - M);
          L += w;
          acc += ((const f32x4*)(P.part_o + r * D))[dq] * w;
        }
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const int head = kvh * G + n % G;
  const int64_t obase = qi * A.out_stride_token + (int64_t)head * D + 4 * dq;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (A.history == 0) ((uint16_t*)A.out)[obase + e] = (uint16_t)q_bits<QT>(acc[e] * inv);
    else ((float*)A.out)[obase + e] = acc[e] * inv;
  }
  if (A.lse != nullptr && dq == 0)
    A.lse[qi * A.num_q_heads + head] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

}  // namespace

}  // namespace oscar

using namespace oscar;

extern "C" int64_t oscar_prefill_workspace_bytes_v1(int64_t history, int64_t num_kv_heads, int64_t head_dim) {
  if (history <= 0) return 0;
  return 2 * history * num_kv_heads * head_dim * (int64_t)sizeof(uint16_t);
}

extern "C" int64_t oscar_prefill_workspace_bytes_v2(int64_t history, int64_t num_tokens, int64_t num_q_heads,
                                                     int64_t num_kv_heads, int64_t head_dim) {
  if (history < 0 || num_tokens < 0 || num_kv_heads < 1 || num_q_heads < num_kv_heads ||
      num_q_heads % num_kv_heads || (head_dim != 128 && head_dim != 256) || num_q_heads / num_kv_heads > kRows)
    return -22;
  const SplitPlan sp = plan_split(history, num_tokens, kRows / (num_q_heads / num_kv_heads), num_kv_heads);
  return hist_bytes(history, num_kv_heads, head_dim) + split_bytes(sp, num_kv_heads, head_dim);
}

extern "C" int oscar_prefill_plan_v1(int64_t history, int64_t num_tokens, int64_t num_q_heads, int64_t num_kv_heads,
                                     int32_t* out, int32_t cap) {
  if (!out || cap < 6 + kMaxChunks + 1 || history < 0 || num_tokens < 0 || num_kv_heads < 1 ||
      num_q_heads < num_kv_heads || num_q_heads % num_kv_heads || num_q_heads / num_kv_heads > kRows)
    return -22;
  const SplitPlan sp = plan_split(history, num_tokens, kRows / (num_q_heads / num_kv_heads), num_kv_heads);
  const int64_t head[6] = {sp.chunks, sp.U, sp.ntq, sp.qmin1, sp.units, sp.slots};
  for (int i = 0; i < 6; ++i) out[i] = (int32_t)head[i];
  for (int c = 0; c <= kMaxChunks; ++c) out[6 + c] = sp.base[c];
  return 0;
}

extern "C" int oscar_attn_prefill_v1(const oscar_prefill_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_attn_prefill_v1: null args");
  const oscar_prefill_args_v1& a = *args;
  if (a.num_tokens == 0) return 0;
  const int64_t D = a.head_dim;
  if (D != 128 && D != 256) return fail(-22, "oscar_attn_prefill_v1: head_dim %lld unsupported", (long long)D);
  if (!a.q || !a.k || !a.v || !a.out || a.num_tokens < 0 || a.num_kv_heads < 1 ||
      a.num_q_heads % a.num_kv_heads)
    return fail(-22, "oscar_attn_prefill_v1: invalid arguments");
  if (a.q_dtype != OSCAR_BF16 && a.q_dtype != OSCAR_F16)
    return fail(-22, "oscar_attn_prefill_v1: q_dtype must be OSCAR_BF16 or OSCAR_F16");
  const int G = (int)(a.num_q_heads / a.num_kv_heads);
  if (G > kRows) return fail(-22, "oscar_attn_prefill_v1: more than %d query heads per KV head", kRows);
  if (a.history < 0) return fail(-22, "oscar_attn_prefill_v1: negative history");
  if (a.history > 0 && (!a.cache.k || !a.cache.v || !a.block_table_row || a.cache.head_dim != D ||
                        a.cache.block_size < 1))
    return fail(-22, "oscar_attn_prefill_v1: history needs the cache and the block-table row");
  // streaming_attention.py:51-53
  if (a.history > 0 && (a.history + a.cache.block_size - 1) / a.cache.block_size > a.block_table_cols)
    return fail(-22, "oscar_attn_prefill_v1: Block table cannot cover the history");
  // q/k/v rows and the history workspace are read as 16-byte vectors
  if ((((uintptr_t)a.q) & 15) || (((uintptr_t)a.k) & 15) || (((uintptr_t)a.v) & 15) ||
      ((a.q_stride_token * 2) & 15) || ((a.kv_stride_token * 2) & 15))
    return fail(-22, "oscar_attn_prefill_v1: q/k/v rows must be 16-byte aligned");
  // the prefill kernel addresses history and chunk rows with 32-bit element offsets
  if ((a.history + 64) * a.num_kv_heads * D >= (1ll << 31) ||
      (a.num_tokens + 64) * a.kv_stride_token >= (1ll << 31))
    return fail(-22, "oscar_attn_prefill_v1: history or chunk too large for one call");
  const int64_t need = oscar_prefill_workspace_bytes_v1(a.history, a.num_kv_heads, D);
  if (a.history > 0 &&
      (a.workspace == nullptr || a.workspace_bytes < need || (((uintptr_t)a.workspace) & 15)))
    return fail(-22, "oscar_attn_prefill_v1: 16-byte aligned workspace of %lld bytes required", (long long)need);
  PrefillParams p{};
  p.a = a;
  p.has_stage = a.staging != nullptr;
  if (a.staging) p.st = *a.staging;
  p.group = G;
  p.qtok = kRows / G;
  if (a.history > 0) {
    p.hist_k = (uint16_t*)a.workspace;
    p.hist_v = p.hist_k + a.history * a.num_kv_heads * D;
  }
  // the balanced split when the workspace holds its partials (after the history values)
  const SplitPlan sp = plan_split(a.history, a.num_tokens, p.qtok, a.num_kv_heads);
  const int64_t hbytes = hist_bytes(a.history, a.num_kv_heads, D), sbytes = split_bytes(sp, a.num_kv_heads, D);
  p.ntq = (int)((a.num_tokens + p.qtok - 1) / p.qtok);
  if (sbytes > 0 && a.workspace != nullptr && (((uintptr_t)a.workspace) & 15) == 0 &&
      a.workspace_bytes >= hbytes + sbytes) {
    p.split = 1;
    p.chunks = sp.chunks;
    p.U = sp.U;
    p.qmin1 = sp.qmin1;
    for (int c = 0; c <= kMaxChunks; ++c) p.base[c] = sp.base[c];
    p.part_o = (float*)((char*)a.workspace + hbytes);
    p.part_lse = p.part_o + sp.slots * a.num_kv_heads * kRows * D;
  }
  hipStream_t s = (hipStream_t)stream;
  if (a.history > 0) {
    const unsigned hb = (unsigned)((a.history * a.num_kv_heads + 3) / 4);
    if (a.q_dtype == OSCAR_F16) {
      if (D == 256) hipLaunchKernelGGL((history_bf16_kernel<256, OSCAR_F16>), dim3(hb), dim3(256), 0, s, p);
      else hipLaunchKernelGGL((history_bf16_kernel<128, OSCAR_F16>), dim3(hb), dim3(256), 0, s, p);
    } else {
      if (D == 256) hipLaunchKernelGGL((history_bf16_kernel<256, OSCAR_BF16>), dim3(hb), dim3(256), 0, s, p);
      else hipLaunchKernelGGL((history_bf16_kernel<128, OSCAR_BF16>), dim3(hb), dim3(256), 0, s, p);
    }
    OSCAR_CHECK_LAUNCH("history_bf16_kernel");
  }
  dim3 grid((unsigned)(p.split ? sp.units : p.ntq), (unsigned)a.num_kv_heads);
  if (a.q_dtype == OSCAR_F16) {
    if (D == 256) hipLaunchKernelGGL((prefill_kernel<256, OSCAR_F16>), grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL((prefill_kernel<128, OSCAR_F16>), grid, dim3(kThreads), 0, s, p);
  } else {
    if (D == 256) hipLaunchKernelGGL((prefill_kernel<256, OSCAR_BF16>), grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL((prefill_kernel<128, OSCAR_BF16>), grid, dim3(kThreads), 0, s, p);
  }
  OSCAR_CHECK_LAUNCH("prefill_kernel");
  if (p.split) {
    const dim3 mgrid((unsigned)((p.ntq - p.qmin1) * (kRows / (256 / (D / 4)))), (unsigned)a.num_kv_heads);
    if (a.q_dtype == OSCAR_F16) {
      if (D == 256) hipLaunchKernelGGL((prefill_merge_kernel<256, OSCAR_F16>), mgrid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((prefill_merge_kernel<128, OSCAR_F16>), mgrid, dim3(256), 0, s, p);
    } else {
      if (D == 256) hipLaunchKernelGGL((prefill_merge_kernel<256, OSCAR_BF16>), mgrid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((prefill_merge_kernel<128, OSCAR_BF16>), mgrid, dim3(256), 0, s, p);
    }
    OSCAR_CHECK_LAUNCH("prefill_merge_kernel");
  }
  return 0;
}
