// Native decode step: the impl's forward for decode-shaped batches in one host call.
//
// Replaces the Python orchestration of oscar_ascend/backend.py:249-393 (forward ->
// write + window -> _streaming_attention -> inverse rotation) for batches whose
// requests all have history (chunks of more than 32 rows per KV head run as sub-requests
// of the split-K decode, up to kMaxSplitRows).  Per call: classify the
// batch from the host metadata, build the split-K plan (oscar_attn_plan_v1) straight
// into a pinned ring slot next to the request table, one host-to-device copy of the
// slot, then the store (or the query rotation), the split-K decode + merge and the
// inverse rotation, all through the public entry points, on the caller's stream (the
// store and decode as oscar_decode_write_v1).
#include <mutex>
#include <vector>

#include "common.h"

namespace oscar {
namespace {

constexpr int kRingSlots = 32;
// longest current chunk (rows per KV head) of a request the step takes: more rows go to
// the prefill path, which decodes the history once for all of its query tiles
constexpr int64_t kMaxSplitRows = 32 * 512;
constexpr int64_t kSlotBytes = 64 << 10;  // request table + plan of up to ~1900 items
constexpr int64_t kAlign = 256;

int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Byte offsets of the step workspace sections.
struct StepLayout {
  int64_t q_rot, k_rot, v_rot, out_rot, lse, partials, total;
  StepLayout(int64_t n, int64_t hq, int64_t hk, int64_t d, int64_t items) {
    int64_t o = 0;
    q_rot = o;    o = align_up(o + n * hq * d * 2, kAlign);
    k_rot = o;    o = align_up(o + n * hk * d * 2, kAlign);
    v_rot = o;    o = align_up(o + n * hk * d * 2, kAlign);
    out_rot = o;  o = align_up(o + n * hq * d * 4, kAlign);
    lse = o;      o = align_up(o + n * hq * 4, kAlign);
    partials = o; o = align_up(o + items * 32 * (d + 1) * 4, kAlign);
    total = o;
  }
};

}  // namespace
}  // namespace oscar

using namespace oscar;

struct oscar_context_v1 {
  int device = -1;
  int cu_count = 0;
  uint8_t* host_ring = nullptr;    // pinned
  uint8_t* dev_ring = nullptr;
  hipEvent_t done[kRingSlots] = {};
  bool used[kRingSlots] = {};
  int next = 0;
  std::mutex mu;
};

extern "C" int oscar_context_create_v1(int32_t device, oscar_context_v1** out) {
  if (!out) return fail(-22, "oscar_context_create_v1: null output");
  *out = nullptr;
  int prev = -1;
  if (hipGetDevice(&prev) != hipSuccess) return fail(-5, "oscar_context_create_v1: no HIP device");
  if (hipSetDevice(device) != hipSuccess) return fail(-22, "oscar_context_create_v1: bad device %d", device);
  auto* c = new oscar_context_v1();
  c->device = device;
  int rc = 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) rc = fail(-5, "oscar_context_create_v1: device properties");
  else c->cu_count = prop.multiProcessorCount;
  if (!rc && hipHostMalloc((void**)&c->host_ring, kRingSlots * kSlotBytes, hipHostMallocDefault) != hipSuccess)
    rc = fail(-12, "oscar_context_create_v1: pinned ring allocation failed");
  if (!rc && hipMalloc((void**)&c->dev_ring, kRingSlots * kSlotBytes) != hipSuccess)
    rc = fail(-12, "oscar_context_create_v1: device ring allocation failed");
  for (int i = 0; !rc && i < kRingSlots; ++i)
    if (hipEventCreateWithFlags(&c->done[i], hipEventDisableTiming) != hipSuccess)
      rc = fail(-12, "oscar_context_create_v1: event creation failed");
  (void)hipSetDevice(prev);  // restore the caller's device (best effort)
  if (rc) {
    oscar_context_destroy_v1(c);
    return rc;
  }
  *out = c;
  return 0;
}

extern "C" int oscar_context_destroy_v1(oscar_context_v1* c) {
  if (!c) return 0;
  // teardown is best effort: a failing call leaves nothing more to release
  int prev = -1;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(c->device);
  for (int i = 0; i < kRingSlots; ++i) {
    if (c->done[i]) {
      (void)hipEventSynchronize(c->done[i]);
      (void)hipEventDestroy(c->done[i]);
    }
  }
  if (c->dev_ring) (void)hipFree(c->dev_ring);
  if (c->host_ring) (void)hipHostFree(c->host_ring);
  (void)hipSetDevice(prev);
  delete c;
  return 0;
}

extern "C" int64_t oscar_step_workspace_bytes_v1(int64_t num_tokens, int64_t num_q_heads,
                                                 int64_t num_kv_heads, int64_t head_dim,
                                                 int64_t num_items) {
  return StepLayout(num_tokens, num_q_heads, num_kv_heads, head_dim, num_items).total;
}

extern "C" int oscar_decode_step_v1(oscar_context_v1* ctx, oscar_step_args_v1* args, void* stream) {
  if (!ctx || !args) return fail(-22, "oscar_decode_step_v1: null context or args");
  oscar_step_args_v1& a = *args;
  a.workspace_needed = 0;
  const int64_t n = a.num_tokens, hq = a.num_q_heads, hk = a.cache.num_kv_heads, d = a.cache.head_dim;
  const int B = a.num_reqs;
  if (n <= 0 || B <= 0 || hk < 1 || hq % hk || !a.host_query_start_loc || !a.host_seq_lens || !a.query ||
      !a.output || !a.block_table || !a.workspace || !a.rk || !a.rv)
    return fail(-22, "oscar_decode_step_v1: invalid arguments");
  if (a.q_dtype != OSCAR_BF16 && a.q_dtype != OSCAR_F16)
    return fail(-22, "oscar_decode_step_v1: q_dtype must be OSCAR_BF16 or OSCAR_F16");
  const bool has_new = a.key != nullptr;
  if (has_new != (a.value != nullptr)) return fail(-22, "oscar_decode_step_v1: key and value go together");
  if (has_new && !a.slot_mapping) return fail(-22, "oscar_decode_step_v1: slot_mapping required with new K/V");
  const int G = (int)(hq / hk);
  if (G > 32) return OSCAR_STEP_NOT_DECODE;  // no 32-row tile holds one token's heads
  const int64_t bs = a.cache.block_size;
  if (bs < 1) return fail(-22, "oscar_decode_step_v1: invalid cache geometry");
  // streaming_attention.py:48-65: table rows for every request, a staging arena of at
  // least one row
  if (a.block_table_rows < B || a.block_table_cols < 1)
    return fail(-22, "Missing request block-table rows");
  if (a.staging != nullptr && a.staging->rows < 1) return fail(-22, "Invalid streaming staging geometry");
  // ---- classify: every request decode-shaped, the requests tile [0, n)
  const int32_t* qsl = a.host_query_start_loc;
  const int32_t* seqs = a.host_seq_lens;
  auto clip = [&](int64_t x) { return x < n ? x : n; };
  for (int r = 0; r < B; ++r) {
    const int64_t q0 = clip(qsl[r]), q1 = clip(qsl[r + 1]);
    if (q1 < q0) return fail(-22, "oscar_decode_step_v1: query_start_loc must be non-decreasing");
    if (seqs[r] < 0) return fail(-22, "oscar_decode_step_v1: negative sequence length");
    const int64_t nq = q1 - q0;
    if (nq == 0) continue;
    if (has_new && seqs[r] < nq) return fail(-22, "oscar_decode_step_v1: sequence length must cover its query chunk");
    // the pages of the history this request reads through the table
    const int64_t hist = has_new ? seqs[r] - nq : seqs[r];
    if ((hist + bs - 1) / bs > a.block_table_cols) return fail(-22, "Block table cannot cover the history");
  }
  if (qsl[0] != 0 || clip(qsl[B]) != n) return OSCAR_STEP_NOT_DECODE;
  for (int r = 0; r < B; ++r) {
    const int64_t nq = clip(qsl[r + 1]) - clip(qsl[r]);
    if (nq == 0) continue;
    // chunks of more than 32 rows per KV head run as sub-requests, up to kMaxSplitRows
    if (has_new && nq * G > kMaxSplitRows) return OSCAR_STEP_NOT_DECODE;
    if (has_new && seqs[r] == nq) return OSCAR_STEP_NOT_DECODE;  // history-free: prefill
  }
  hipStream_t s = (hipStream_t)stream;
  // the plan is built on the host at every call and copied from a ring slot that later
  // calls rewrite: a captured copy would replay stale metadata
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess)
    return fail(-5, "oscar_decode_step_v1: cannot query the stream's capture status");
  if (cap != hipStreamCaptureStatusNone)
    return fail(-22, "oscar_decode_step_v1: eager only (the stream is capturing a graph)");
  // ---- ring slot (wait only if the slot's previous call has not finished reading it)
  std::unique_lock<std::mutex> lock(ctx->mu);
  const int slot = ctx->next;
  ctx->next = (ctx->next + 1) % kRingSlots;
  if (ctx->used[slot] && hipEventSynchronize(ctx->done[slot]) != hipSuccess)
    return fail(-5, "oscar_decode_step_v1: ring event wait failed");
  uint8_t* host = ctx->host_ring + slot * kSlotBytes;
  uint8_t* dev = ctx->dev_ring + slot * kSlotBytes;
  // slot layout: qsl [B + 1] (clipped) | seqs [B] | groups | items
  // groups: (sub-)requests of 32 / G query tokens x kv heads
  int64_t ngroups = 0;
  for (int r = 0; r < B; ++r) ngroups += (clip(qsl[r + 1]) - clip(qsl[r]) + 32 / G - 1) / (32 / G) * hk;
  const int64_t o_seqs = align_up((int64_t)(B + 1) * 4, 16);
  const int64_t o_groups = align_up(o_seqs + (int64_t)B * 4, 16);
  const int64_t o_items = align_up(o_groups + (int64_t)ngroups * OSCAR_GROUP_INTS * 4, 16);
  if (o_items + OSCAR_WORK_INTS * 4 > kSlotBytes) return OSCAR_STEP_NOT_DECODE;  // too many requests for a slot
  const int max_groups = (int)ngroups;
  int32_t* h_qsl = (int32_t*)host;
  for (int r = 0; r <= B; ++r) h_qsl[r] = (int32_t)clip(qsl[r]);
  int32_t* h_seqs = (int32_t*)(host + o_seqs);
  for (int r = 0; r < B; ++r) h_seqs[r] = seqs[r];
  int32_t* h_groups = (int32_t*)(host + o_groups);
  int32_t* h_items = (int32_t*)(host + o_items);
  const int max_items = (int)((kSlotBytes - o_items) / (OSCAR_WORK_INTS * 4));
  const bool window = a.staging != nullptr;
  oscar_plan_v1 plan{};
  const int target = a.target_items > 0 ? a.target_items : ctx->cu_count;
  int rc = oscar_attn_plan_v1(h_qsl, h_seqs, B, has_new, (int32_t)hk, G, (int32_t)d, 8192, target,
                              window ? a.sink_tokens_eff : 0, window ? a.recent_tokens : 0, h_items, max_items,
                              h_groups, max_groups, &plan);
  if (rc == -28) return OSCAR_STEP_NOT_DECODE;  // a plan larger than a ring slot: the general path
  if (rc < 0) return rc;
  const StepLayout L(n, hq, hk, d, plan.num_items);
  if (a.workspace_bytes < L.total) {
    a.workspace_needed = L.total;
    return fail(-28, "oscar_decode_step_v1: workspace of %lld bytes < %lld", (long long)a.workspace_bytes,
                (long long)L.total);
  }
  const int64_t used = o_items + (int64_t)plan.num_items * OSCAR_WORK_INTS * 4;
  if (hipMemcpyAsync(dev, host, used, hipMemcpyHostToDevice, s) != hipSuccess)
    return fail(-5, "oscar_decode_step_v1: metadata copy failed");
  ctx->used[slot] = true;
  const int32_t* d_qsl = (const int32_t*)dev;
  const int32_t* d_seqs = (const int32_t*)(dev + o_seqs);
  uint8_t* ws = (uint8_t*)a.workspace;
  void* q_rot = ws + L.q_rot;
  void* k_rot = ws + L.k_rot;
  void* v_rot = ws + L.v_rot;
  float* out_rot = (float*)(ws + L.out_rot);
  float* lse = (float*)(ws + L.lse);
  // ---- write (enqueued with the decode below) or the query rotation alone
  rc = 0;
  oscar_store_args_v1 st{};
  if (has_new) {
    st.key = a.key;
    st.value = a.value;
    st.kv_dtype = a.q_dtype;
    st.num_tokens = n;
    st.key_stride_token = st.value_stride_token = a.kv_stride_token;
    st.query = a.query;
    st.num_q_heads = hq;
    st.query_stride_token = hq * d;
    st.rk = a.rk;
    st.rv = a.rv;
    st.k_clip_ratio = a.k_clip_ratio;
    st.v_clip_ratio = a.v_clip_ratio;
    st.slot_mapping = a.slot_mapping;
    st.cache = a.cache;
    st.stage_mode = window ? a.stage_mode : OSCAR_STAGE_NONE;
    if (window) st.staging = *a.staging;
    st.query_start_loc = d_qsl;
    st.seq_lens = d_seqs;
    st.num_reqs = B;
    st.recent_tokens = a.recent_tokens;
    st.sink_tokens_eff = a.sink_tokens_eff;
    st.query_rot = q_rot;
    st.key_rot = k_rot;
    st.value_rot = v_rot;
    st.slot_claims = a.slot_claims;
    st.seat_claims = a.seat_claims;
    st.epoch_counter = a.epoch_counter;
    st.workspace = a.store_workspace;
    st.workspace_bytes = a.store_workspace_bytes;
    st.arrivals = a.arrivals;
  } else {
    oscar_rotate_args_v1 ro{};
    ro.x = a.query;
    ro.x_dtype = a.q_dtype;
    ro.rows = n * hq;
    ro.x_stride_row = d;
    ro.r = a.rk;
    ro.out = q_rot;
    ro.out_dtype = a.q_dtype;
    ro.out_stride_row = d;
    ro.head_dim = d;
    rc = oscar_rotate_v1(&ro, stream);
  }
  // ---- read: split-K decode + merge, then out_rot @ R_v^T into the output
  if (rc == 0) {
    oscar_attn_args_v1 at{};
    at.q = q_rot;
    at.num_tokens = n;
    at.num_q_heads = hq;
    at.q_stride_token = hq * d;
    if (has_new) {
      at.k_new = k_rot;
      at.v_new = v_rot;
      at.kv_new_stride_token = hk * d;
    }
    at.cache = a.cache;
    at.block_table = a.block_table;
    at.block_table_stride = a.block_table_stride;
    at.block_table_rows = a.block_table_rows;
    at.block_table_cols = a.block_table_cols;
    at.query_start_loc = d_qsl;
    at.seq_lens = d_seqs;
    at.num_reqs = B;
    at.staging = a.staging;
    at.scale = a.scale;
    at.items = (const int32_t*)(dev + o_items);
    at.num_items = plan.num_items;
    at.groups = (const int32_t*)(dev + o_groups);
    at.num_groups = plan.num_groups;
    at.workspace = ws + L.partials;
    at.workspace_bytes = L.total - L.partials;
    at.max_group_items = plan.max_group_items;
    at.out_rot = out_rot;
    at.lse = lse;
    at.q_dtype = a.q_dtype;
    // with new tokens: the store and the decode in one call (a small store's
    // quantization and slot / window writes ride in the decode's merge launch)
    rc = has_new ? oscar_decode_write_v1(&st, &at, stream) : oscar_attn_decode_v1(&at, stream);
  }
  if (rc == 0) {
    oscar_rotate_args_v1 ro{};
    ro.x = out_rot;
    ro.x_dtype = OSCAR_F32;
    ro.rows = n * hq;
    ro.x_stride_row = d;
    ro.r = a.rv;
    ro.transpose = 1;
    ro.out = a.output;
    ro.out_dtype = a.q_dtype;
    ro.out_stride_row = d;
    ro.head_dim = d;
    rc = oscar_rotate_v1(&ro, stream);
  }
  // the slot may be rewritten once everything enqueued above has run
  if (hipEventRecord(ctx->done[slot], s) != hipSuccess && rc == 0)
    rc = fail(-5, "oscar_decode_step_v1: event record failed");
  return rc;
}
