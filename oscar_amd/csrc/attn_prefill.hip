// Causal GQA prefill over an optional INT2 history for gfx950 (MFMA bf16).
//
// Replaces oscar_ascend/kernels/prefill.py:69-72 / decode_kernel.py:70-117
// (fresh-only prefill: causal SDPA of the current chunk, original domain, bf16 out)
// and the long-continuation use of slab_attention.py:376-476 (history waves plus
// the causal current chunk, rotated domain, fp32 out + LSE).
//
// Query i (0-based in the chunk) sees keys [0, history + i + 1).  A workgroup of
// four waves owns 128 query rows (rows = tokens x heads of one KV head, GQA
// packed); key tiles of 32 are staged in LDS as bf16 values with the reference
// rounding (history: q_dtype(fp16(code*scale + zero)) or the staged fp32 value when
// the seat's owner tag matches; current chunk: the given bf16 values) and shared
// by the four waves.  Each wave: S^T = K Q^T (v_mfma_f32_32x32x16_bf16), online
// softmax in fp32 (log2 domain), O^T += V^T P^T with V^T read from LDS by
// ds_read_b64_tr_b16.
#include "common.h"

namespace oscar {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 256;
constexpr int kKeys = 32;
constexpr int kRows = 128;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
typedef short __attribute__((ext_vector_type(4))) i16x4;

__device__ __forceinline__ float round_hist_bf16(float x) {
  float h = __half2float(__float2half_rn(x));
  return bf16_bits_to_f32(f32_to_bf16_bits(h));
}

struct PrefillParams {
  oscar_prefill_args_v1 a;
  oscar_staging_v1 st;
  int has_stage;
  int group;
  int qtok;  // query tokens per workgroup
};

template <int D>
__global__ __launch_bounds__(kThreads, 1) void prefill_kernel(PrefillParams P) {
  const oscar_prefill_args_v1& A = P.a;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 31, g = lane >> 5;
  const int G = P.group;
  const int ntiles_q = (int)((A.num_tokens + P.qtok - 1) / P.qtok);
  const int qt = ntiles_q - 1 - (int)blockIdx.x;  // heaviest (latest) query tiles first
  const int kvh = blockIdx.y;
  const int64_t q0 = (int64_t)qt * P.qtok;
  const int64_t q1 = (q0 + P.qtok < A.num_tokens) ? q0 + P.qtok : A.num_tokens;
  const int64_t hist = A.history;
  const int64_t nkeys = hist + q1;  // keys visible to the last query of the tile

  // rows padded by 16 bytes so that 16-byte reads of consecutive keys hit distinct banks
  __shared__ __attribute__((aligned(16))) uint16_t s_k[kKeys][D + 8];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kKeys][D + 8];

  // this lane's row
  const int n = wave * 32 + m;
  const int64_t qi = q0 + n / G;
  const bool row_ok = (n < P.qtok * G) && (qi < q1);
  const int head = kvh * G + n % G;
  const uint16_t* qrow = (const uint16_t*)A.q + (row_ok ? qi : 0) * A.q_stride_token + (int64_t)head * D;
  bf16x8 qb[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      qb[j][e] = __builtin_bit_cast(__bf16, (unsigned short)(row_ok ? qrow[16 * j + 8 * g + e] : 0));
  const float c = A.scale * kLog2e;
  const int64_t limit = hist + qi + 1;  // keys [0, limit) visible to this row

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 O[D / 32];
#pragma unroll
  for (int b = 0; b < D / 32; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[b][r] = 0.f;

  const int64_t bs = A.cache.block_size;
  const int64_t hk = A.num_kv_heads;
  const int ktiles = (int)((nkeys + kKeys - 1) / kKeys);
  for (int kt = 0; kt < ktiles; ++kt) {
    const int64_t k0 = (int64_t)kt * kKeys;
    __syncthreads();
    // ---- fill: thread -> (key, 8 d-chunks of D/8)
    {
      const int kk = tid >> 3, dc = tid & 7;
      const int64_t p = k0 + kk;
      constexpr int W = D / 8;
      float kv[W], vv[W];
      if (p < hist) {
        int64_t blk = A.block_table_row[p / bs];
        if (blk < 0 || blk >= A.cache.num_blocks) blk = 0;  // host validates; never fault
        const int64_t off = p % bs;
        bool staged = false;
        const int64_t seat = P.has_stage ? (blk % P.st.rows) * bs + off : 0;
        if (P.has_stage) staged = P.st.owner[seat] == blk;
        if (staged) {
          const float* sk = P.st.stage_k + (seat * hk + kvh) * D + dc * W;
          const float* sv = P.st.stage_v + (seat * hk + kvh) * D + dc * W;
#pragma unroll
          for (int i = 0; i < W; ++i) { kv[i] = round_hist_bf16(sk[i]); vv[i] = round_hist_bf16(sv[i]); }
        } else {
          const uint8_t* ks = A.cache.k + blk * A.cache.k_stride[0] + off * A.cache.k_stride[1] + kvh * A.cache.k_stride[2];
          const uint8_t* vs = A.cache.v + blk * A.cache.v_stride[0] + off * A.cache.v_stride[1] + kvh * A.cache.v_stride[2];
          const unsigned m0 = *(const unsigned*)ks, m1 = *(const unsigned*)(ks + 4);
          const float sk = f16_bits_to_f32(m0 & 0xffff), zk = f16_bits_to_f32(m0 >> 16);
          const float sv = f16_bits_to_f32(m1 & 0xffff), zv = f16_bits_to_f32(m1 >> 16);
#pragma unroll
          for (int i = 0; i < W; i += 4) {
            const unsigned kb = ks[32 + (dc * W + i) / 4], vb = vs[(dc * W + i) / 4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              kv[i + j] = round_hist_bf16(__fadd_rn(__fmul_rn((float)((kb >> (2 * j)) & 3u), sk), zk));
              vv[i + j] = round_hist_bf16(__fadd_rn(__fmul_rn((float)((vb >> (2 * j)) & 3u), sv), zv));
            }
          }
        }
      } else if (p < nkeys) {
        const int64_t ci = p - hist;  // current-chunk index
        const uint16_t* kn = (const uint16_t*)A.k + ci * A.kv_stride_token + kvh * D + dc * W;
        const uint16_t* vn = (const uint16_t*)A.v + ci * A.kv_stride_token + kvh * D + dc * W;
#pragma unroll
        for (int i = 0; i < W; ++i) { kv[i] = bf16_bits_to_f32(kn[i]); vv[i] = bf16_bits_to_f32(vn[i]); }
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) { kv[i] = 0.f; vv[i] = 0.f; }
      }
#pragma unroll
      for (int i = 0; i < W; i += 8) {
        u32x4 kw, vw;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kw[j] = (unsigned)f32_to_bf16_bits(kv[i + 2 * j]) | ((unsigned)f32_to_bf16_bits(kv[i + 2 * j + 1]) << 16);
          vw[j] = (unsigned)f32_to_bf16_bits(vv[i + 2 * j]) | ((unsigned)f32_to_bf16_bits(vv[i + 2 * j + 1]) << 16);
        }
        *(u32x4*)&s_k[kk][dc * W + i] = kw;
        *(u32x4*)&s_v[kk][dc * W + i] = vw;
      }
    }
    __syncthreads();
    // ---- S^T = K Q^T
    f32x16 S = {};
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      const bf16x8 ka = *(const bf16x8*)&s_k[m][16 * j + 8 * g];
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qb[j], S, 0, 0, 0);
    }
    const bool full = (k0 + kKeys <= hist + q0 + 1);  // visible to every row of the tile
    float xs[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t p = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
      const bool vis = row_ok && (full || p < limit);
      xs[r] = vis ? S[r] * c : -INFINITY;
      mx = fmaxf(mx, xs[r]);
    }
    {
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const float m_new = fmaxf(m_run, mx);
    if (__any(m_new > m_run)) {
      const float f = (m_new == m_run) ? 1.f : (m_run == -INFINITY ? 0.f : exp2f(m_run - m_new));
#pragma unroll
      for (int b = 0; b < D / 32; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[b][r] *= f;
      l_run *= f;
    }
    m_run = m_new;
    bf16x8 pb[2];
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = (xs[r] == -INFINITY) ? 0.f : exp2f(xs[r] - m_run);
      lsum += pr;
      pb[r >> 3][r & 7] = __builtin_bit_cast(__bf16, f32_to_bf16_bits(pr));
    }
    l_run += lsum;
    // ---- O^T += V^T P^T; A operand (V^T) via transpose reads of s_v
    const int G16 = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int b = 0; b < D / 32; ++b) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bf16x8 va;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = 16 * s + 4 * (G16 >> 1) + 8 * h + (i16 >> 2);
          const uint16_t* addr = &s_v[key][32 * b + 16 * (G16 & 1) + 4 * (i16 & 3)];
          auto t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(addr));
#pragma unroll
          for (int e = 0; e < 4; ++e) va[4 * h + e] = __builtin_bit_cast(__bf16, (unsigned short)t[e]);
        }
        O[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[s], O[b], 0, 0, 0);
      }
    }
  }
  // ---- finalize: row n = lane's row; O^T block b register r holds d = 32b + out_row(r, g)
  float l_tot;
  {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_tot = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (!row_ok) return;
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  const int64_t obase = qi * A.out_stride_token + (int64_t)head * D;
#pragma unroll
  for (int b = 0; b < D / 32; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * b + 8 * (r >> 2) + 4 * g + (r & 3);
      const float v = O[b][r] * inv;
      if (hist == 0) ((uint16_t*)A.out)[obase + d] = f32_to_bf16_bits(v);
      else ((float*)A.out)[obase + d] = v;
    }
  if (A.lse != nullptr && g == 0)
    A.lse[qi * A.num_q_heads + head] = (l_tot > 0.f) ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
}

}  // namespace

}  // namespace oscar

using namespace oscar;

extern "C" int oscar_attn_prefill_v1(const oscar_prefill_args_v1* args, void* stream) {
  if (!args) return fail(-22, "oscar_attn_prefill_v1: null args");
  const oscar_prefill_args_v1& a = *args;
  if (a.num_tokens == 0) return 0;
  const int64_t D = a.head_dim;
  if (D != 128 && D != 256) return fail(-22, "oscar_attn_prefill_v1: head_dim %lld unsupported", (long long)D);
  if (!a.q || !a.k || !a.v || !a.out || a.num_tokens < 0 || a.num_kv_heads < 1 ||
      a.num_q_heads % a.num_kv_heads)
    return fail(-22, "oscar_attn_prefill_v1: invalid arguments");
  const int G = (int)(a.num_q_heads / a.num_kv_heads);
  if (G > kRows) return fail(-22, "oscar_attn_prefill_v1: more than %d query heads per KV head", kRows);
  if (a.history < 0) return fail(-22, "oscar_attn_prefill_v1: negative history");
  if (a.history > 0 && (!a.cache.k || !a.cache.v || !a.block_table_row || a.cache.head_dim != D))
    return fail(-22, "oscar_attn_prefill_v1: history needs the cache and the block-table row");
  PrefillParams p{};
  p.a = a;
  p.has_stage = a.staging != nullptr;
  if (a.staging) p.st = *a.staging;
  p.group = G;
  p.qtok = kRows / G;
  const int ntq = (int)((a.num_tokens + p.qtok - 1) / p.qtok);
  dim3 grid(ntq, (unsigned)a.num_kv_heads);
  hipStream_t s = (hipStream_t)stream;
  if (D == 256) hipLaunchKernelGGL(prefill_kernel<256>, grid, dim3(kThreads), 0, s, p);
  else hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kThreads), 0, s, p);
  OSCAR_CHECK_LAUNCH("prefill_kernel");
  return 0;
}
