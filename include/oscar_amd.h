/*
 * oscar_amd.h -- C ABI of the MI355X (gfx950) OSCAR INT2 rotated KV-cache path.
 *
 * Plain C: device pointers, byte strides, shapes and a HIP stream passed as
 * void*.  No torch types.  Every entry point validates its arguments on the
 * host, launches asynchronously on `stream`, allocates nothing (scratch memory
 * is caller-provided) and returns 0 or a negative errno-style status; the
 * message for the last failure on the calling thread is returned by
 * oscar_last_error().
 *
 * Reference interfaces replaced (jpl123123/oscar, Python/Triton-Ascend):
 *   oscar_store_v1       oscar_ascend/kernels/store_kernel.py:54-102 (oscar_store_ref)
 *                        and :247-279 (oscar_store_triton), fused with
 *                        oscar_ascend/backend.py:130-148 (_rotate_clip),
 *                        :151-198 (do_kv_cache_update tag invalidation) and
 *                        :513-555 (_staging_write window + owner tags), plus the
 *                        read-path rotations of backend.py:370-373.
 *   oscar_rotate_v1      oscar_ascend/backend.py:371 (q @ R_k) and :382
 *                        (out_rot @ R_v^T) -- dense D x D rotation.
 *   oscar_attn_plan_v1   oscar_ascend/kernels/slab_attention.py:31-92
 *                        (plan_slabs / slab_steps host planning).
 *   oscar_attn_decode_v1 oscar_ascend/kernels/slab_attention.py:376-476
 *                        (slab_attention: history waves + current chunk + LSE merge).
 *   oscar_attn_prefill_v1 oscar_ascend/kernels/prefill.py:69-72 (oscar_prefill,
 *                        fresh-only causal prefill) and the long-continuation use of
 *                        slab_attention (history + causal current chunk).
 *
 * A maintainer binds these from the reference's Python backend with ctypes
 * (see INTEGRATION.md); oscar_amd/_lib.py is that binding.
 */
#ifndef OSCAR_AMD_H
#define OSCAR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OSCAR_ABI_VERSION 3

/* element types of dense inputs/outputs */
enum oscar_dtype { OSCAR_F32 = 0, OSCAR_F16 = 1, OSCAR_BF16 = 2 };

/* Packed INT2 paged cache pair, addressed as bytes (cache.view(uint8)).
 * Slot layout (oscar_ascend/format.py:19-38): K slot [0:8] = K scale, K zero,
 * V scale, V zero (fp16 little endian), [32:32+D/4] = K codes; V slot
 * [0:D/4] = V codes.  Strides are in bytes: block, token-in-block, kv head. */
typedef struct oscar_cache_v1 {
  uint8_t* k;
  uint8_t* v;
  int64_t num_blocks;
  int64_t block_size;
  int64_t num_kv_heads;
  int64_t head_dim;
  int64_t k_stride[3];
  int64_t v_stride[3];
} oscar_cache_v1;

/* FP32 sink/recent staging window (backend.py:492-511).  stage_k/stage_v are
 * contiguous [rows, block_size, num_kv_heads, head_dim] fp32; owner is
 * contiguous [rows, block_size] int64 (-1 = empty, else physical block id). */
typedef struct oscar_staging_v1 {
  float* stage_k;
  float* stage_v;
  int64_t* owner;
  int64_t rows;
} oscar_staging_v1;

enum oscar_stage_mode {
  OSCAR_STAGE_NONE = 0,       /* no staging arena: plain INT2 store */
  OSCAR_STAGE_INVALIDATE = 1, /* standalone KV update: owner[seat] = -1 for written seats */
  OSCAR_STAGE_WRITE = 2       /* forward: last writer per seat sets owner (keep ? block : -1)
                                 and kept seats receive the unclipped fp32 rotated K/V */
};

typedef struct oscar_store_args_v1 {
  /* new tokens: key/value [num_tokens, num_kv_heads, head_dim], row stride in elements */
  const void* key;
  const void* value;
  int32_t kv_dtype;             /* OSCAR_BF16 / OSCAR_F16 / OSCAR_F32 */
  int64_t num_tokens;
  int64_t key_stride_token;
  int64_t value_stride_token;
  /* optional query [num_tokens, num_q_heads, head_dim] to rotate for the read path */
  const void* query;            /* may be NULL */
  int64_t num_q_heads;
  int64_t query_stride_token;
  /* rotations [head_dim, head_dim] fp32 row-major (x_rot = x @ R); NULL = identity */
  const float* rk;
  const float* rv;
  float k_clip_ratio;           /* 0 disables the sort-based clip */
  float v_clip_ratio;
  const int64_t* slot_mapping;  /* [num_tokens]; negative = skip */
  oscar_cache_v1 cache;
  /* staging */
  int32_t stage_mode;           /* enum oscar_stage_mode */
  oscar_staging_v1 staging;
  const int32_t* query_start_loc; /* [num_reqs + 1] device, clipped to num_tokens */
  const int32_t* seq_lens;        /* [num_reqs] device */
  int32_t num_reqs;
  int32_t recent_tokens;
  int32_t sink_tokens_eff;        /* (sink // block_size) * block_size */
  /* optional read-path outputs in kv_dtype, contiguous [num_tokens, H, head_dim] */
  void* query_rot;              /* x @ R_k for the queries (may be NULL) */
  void* key_rot;                /* x @ R_k, unclipped (may be NULL) */
  void* value_rot;              /* x @ R_v, unclipped (may be NULL) */
  /* scratch: last-writer claims, entries (epoch << 24 | token), num_tokens < 2^24;
   * zero-initialised once.
   * The call's epoch is epoch_counter[0] + 1: the first launch of a call of more
   * than 64 tokens stores it in epoch_counter[1], the next copies it to
   * epoch_counter[0], so replays of a captured graph always claim with a fresh epoch
   * (no host round trip).  Calls of <= 64 tokens find last writers by scanning. */
  int64_t* slot_claims;         /* [num_blocks * block_size] */
  int64_t* seat_claims;         /* [rows * block_size] (stage mode 2) */
  int64_t* epoch_counter;       /* device int64[2], zero-initialised once, shared per device */
  /* 16-byte aligned, >= oscar_store_workspace_bytes_v1(num_tokens, num_kv_heads, head_dim):
   * calls of <= 64 tokens pass their fp32 column slices through it; larger calls keep
   * the exact-pass lists, the per-token window flags and the fp16 planes of R_k / R_v */
  void* workspace;
  int64_t workspace_bytes;
  /* calls of <= 64 tokens: uint32 [2 * 64 * num_kv_heads], zero-initialised once and
   * shared per device; one arrival counter per group of 8 K or V vectors uses the
   * first 2 * ceil(num_tokens * num_kv_heads / 8) words (every call leaves them zero;
   * calls that overlap on one device race on them) */
  uint32_t* arrivals;
} oscar_store_args_v1;

int64_t oscar_store_workspace_bytes_v1(int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim);
/* Codes, scales / zeros, slot bytes and owner tags are those of the correctly rounded
 * fp32 rotation.  FP32 window values are that rotation for calls of <= 64 tokens; larger
 * calls store the certified MFMA rotation, within 2^-20 ||x|| ||R_:d|| + 2^-22 |y| of it
 * (bf16 / fp16 inputs; 2^-19 for fp32). */
int oscar_store_v1(const oscar_store_args_v1* args, void* stream);

/* y[M, D] = x[M, D] @ R[D, D] (or @ R^T when transpose != 0); fp32 accumulate
 * of bf16 hi/lo split products (|error| < 2^-16 |x||R|); out in out_dtype. */
typedef struct oscar_rotate_args_v1 {
  const void* x;
  int32_t x_dtype;
  int64_t rows;
  int64_t x_stride_row;         /* elements */
  const float* r;
  int32_t transpose;
  void* out;
  int32_t out_dtype;
  int64_t out_stride_row;       /* elements */
  int64_t head_dim;
} oscar_rotate_args_v1;

int oscar_rotate_v1(const oscar_rotate_args_v1* args, void* stream);

/* Work planning for the split-K decode (host function, no device access).
 * qsl/seqs are host arrays.  Writes up to max_items work items of
 * OSCAR_WORK_INTS int32 each and returns the item count (or < 0); with
 * items == NULL or groups == NULL it only fills *plan (size query).
 *
 * Keys of a (request, kv head) group are cut into 32-token tiles.  sink_tokens
 * and recent_tokens describe the FP32 staging window the store keeps (positions
 * < sink_tokens and >= seq - recent_tokens; 0 = none): a hint for balance only,
 * the decode finds staged tokens from the owner tags whatever the plan expects.
 * The expected window tiles and the tiles at and past the first masked or
 * current key cost more (FP32 rows, one tile at a time); they are dealt to items
 * of their own, the history tiles between them to the others, each range
 * round-robin (item i of k: tiles first + i, first + i + k, ...), or the whole
 * group as one range where that takes fewer items, so that the most expensive
 * item is as cheap as target_items allows, with at most 128 items in a group (one
 * load round of the merge) where the 256-tile item limit allows.  A request with more than 32 rows per
 * kv head (n_q * group > 32; group <= 32) is planned as sub-requests of 32 / group
 * query tokens, each a group of its own: sub-request [a, b) of a request of n_q
 * queries and length seq has seq - n_q + b keys, its query i sees keys
 * [0, seq - n_q + a + i + 1), and with has_new the keys from seq - n_q on are the
 * current chunk's rows (a = the sub-request's offset in the chunk).  Item record,
 * int32[8]:
 *   [0] request  [1] kv_head | n_q << 16  [2] first tile
 *   [3] tile stride (bits 0-11) | offset a in the chunk << 12
 *   [4] tile count  [5] partial slot  [6] first query token  [7] seq length
 * (n_q, first query token and seq length of the sub-request).  Group record,
 * int32[OSCAR_GROUP_INTS]: request, kv head, first partial slot, slot count, first
 * query token, query count, 0, 0. */
#define OSCAR_WORK_INTS 8
#define OSCAR_GROUP_INTS 8
typedef struct oscar_plan_v1 {
  int32_t num_items;
  int32_t num_groups;           /* request x kv-head groups with queries */
  int64_t partial_bytes;        /* workspace bytes needed by oscar_attn_decode_v1 */
  int32_t max_group_items;      /* largest item count of any group (sizes the merge) */
  int32_t reserved;
} oscar_plan_v1;

int oscar_attn_plan_v1(const int32_t* query_start_loc, const int32_t* seq_lens, int32_t num_reqs,
                       int32_t has_new, int32_t num_kv_heads, int32_t group, int32_t head_dim,
                       int32_t chunk_tokens, int32_t target_items, int32_t sink_tokens,
                       int32_t recent_tokens, int32_t* items, int32_t max_items, int32_t* groups,
                       int32_t max_groups, oscar_plan_v1* plan);

typedef struct oscar_attn_args_v1 {
  const void* q;                /* [n, Hq, D] rotated queries in q_dtype */
  int64_t num_tokens;
  int64_t num_q_heads;
  int64_t q_stride_token;       /* elements */
  const void* k_new;            /* [n, Hk, D] rotated current chunk or NULL (cache-only) */
  const void* v_new;
  int64_t kv_new_stride_token;
  oscar_cache_v1 cache;
  const int32_t* block_table;   /* [num_reqs, max_blocks] */
  int64_t block_table_stride;
  const int32_t* query_start_loc; /* device [num_reqs + 1] */
  const int32_t* seq_lens;        /* device [num_reqs] */
  int32_t num_reqs;
  const oscar_staging_v1* staging; /* NULL = no window */
  float scale;
  const int32_t* items;         /* device copy of the plan */
  int32_t num_items;
  const int32_t* groups;
  int32_t num_groups;
  void* workspace;              /* item partials, >= plan.partial_bytes */
  int64_t workspace_bytes;      /* checked: >= num_items * 32 * (D + 1) * 4 */
  int32_t max_group_items;      /* plan.max_group_items (0: num_items) */
  float* out_rot;               /* [n, Hq, D] fp32 rotated output (required) */
  float* lse;                   /* [n, Hq] natural-log LSE (required) */
  int32_t phases;               /* 0 = split-K pass then merge; 1 = split-K pass only;
                                   2 = merge only (the workspace holds the pass) */
  int32_t q_dtype;              /* OSCAR_BF16 or OSCAR_F16: q, k_new, v_new; history values
                                   are rounded q_dtype(fp16(x)) as the reference does */
  /* block_table geometry [rows, cols] (streaming_attention.py:48-53): rows >= num_reqs and
   * cols >= 1 are checked on the host (-22, "Missing request block-table rows").  The
   * lengths are device data here, so coverage (ceil(history / block_size) <= cols) is
   * checked by the kernel: an item whose history needs a column past cols reads no
   * table entry and turns its group's rows into NaN.  The entry points that hold host
   * lengths (oscar_decode_step_v1, oscar_attn_prefill_v1) reject such a table on the
   * host with "Block table cannot cover the history". */
  int64_t block_table_rows;
  int64_t block_table_cols;
} oscar_attn_args_v1;

int oscar_attn_decode_v1(const oscar_attn_args_v1* args, void* stream);

/* A step's store and split-K decode in one call: oscar_store_v1(store) then
 * oscar_attn_decode_v1(attn) on `stream`, except that for a store of <= 64 tokens (and
 * attn->phases == 0, a non-empty plan) the store's quantization, slot bytes, FP32 window
 * copies and owner tags are written by extra workgroups of the decode's merge launch
 * instead of the store's own launch, so the decode starts once the store's rotation has
 * run.  From the rotation to the merge the seats the call writes carry a pending owner tag
 * (-2, which matches no block): the decode sees the window as the store leaves it.  attn
 * reads the store's rotated outputs (q = store->query_rot, k_new / v_new = key_rot /
 * value_rot).  No counterpart in the reference, whose write (backend.py:249-333)
 * completes before its read (:334-393).  Bytes, tags, window values and outputs are the
 * same as oscar_store_v1 then oscar_attn_decode_v1 provided that no valid slot of the
 * store lies inside the history the decode reads (a slot of a page in a request's block
 * table below its history length): the deferred quantization lands after the split-K
 * pass has read the old codes.  vLLM's block allocator gives this (a step writes only
 * the slots of its new tokens, past every history); a caller that rewrites history
 * slots in the same step calls oscar_store_v1 and oscar_attn_decode_v1 instead. */
int oscar_decode_write_v1(const oscar_store_args_v1* store, const oscar_attn_args_v1* attn, void* stream);

/* oscar_attn_decode_v1 that allocates nothing and takes no workspace: the item
 * partials live in a library-owned static device array of
 * OSCAR_DECODE_STATIC_MAX_ITEMS * 32 * 257 * 4 bytes (16.8 MB, held on every device
 * the library runs on until the process ends).  No counterpart in the reference: it
 * is for callers that cannot allocate (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  args->workspace / workspace_bytes are ignored; a plan of
 * more than OSCAR_DECODE_STATIC_MAX_ITEMS items is rejected (-22).  The stream must
 * belong to the current device.  Every call on a device shares that device's array
 * (the split-K pass writes every partial the merge reads, so nothing needs clearing):
 * calls that overlap on one device race, and phases 1 then 2 must not be separated
 * by another call on the device.  The first call on a device looks up the array's
 * address (hipGetSymbolAddress); make it outside graph capture. */
#define OSCAR_DECODE_STATIC_MAX_ITEMS 512
int oscar_attn_decode_static_v1(const oscar_attn_args_v1* args, void* stream);

typedef struct oscar_prefill_args_v1 {
  const void* q;                /* [n, Hq, D] in q_dtype */
  int64_t q_stride_token;
  const void* k;                /* [n, Hk, D] current chunk in q_dtype */
  const void* v;
  int64_t kv_stride_token;
  int64_t num_tokens;
  int64_t num_q_heads;
  int64_t num_kv_heads;
  int64_t head_dim;
  int64_t history;              /* cached prefix length (0 = fresh-only) */
  oscar_cache_v1 cache;         /* used when history > 0 */
  const int32_t* block_table_row; /* [max_blocks] of this request */
  const oscar_staging_v1* staging;
  float scale;
  void* out;                    /* [n, Hq, D]: q_dtype when history == 0, else fp32 rotated */
  int64_t out_stride_token;
  float* lse;                   /* [n, Hq] or NULL */
  /* history > 0: 16-byte aligned scratch for the history's K/V values in q_dtype,
   * >= oscar_prefill_workspace_bytes_v1(history, num_kv_heads, head_dim) */
  void* workspace;
  int64_t workspace_bytes;
  int32_t q_dtype;              /* OSCAR_BF16 or OSCAR_F16: q, k, v (history values are
                                   rounded q_dtype(fp16(x)) as the reference does) */
  /* entries of block_table_row: ceil(history / block_size) > block_table_cols is
   * rejected (-22, "Block table cannot cover the history", streaming_attention.py:48-53) */
  int64_t block_table_cols;
} oscar_prefill_args_v1;

int64_t oscar_prefill_workspace_bytes_v1(int64_t history, int64_t num_kv_heads, int64_t head_dim);
int oscar_attn_prefill_v1(const oscar_prefill_args_v1* args, void* stream);

/* Workspace for oscar_attn_prefill_v1 with the balanced split of the key ranges: the
 * history values (as v1, rounded up to 256 bytes) plus the FP32 partials of the query
 * tiles (128 GQA rows each) whose key range is cut into chunks of about half a compute
 * unit's share of the call's work; a merge launch combines them (FP32 LSE merge,
 * slab_attention.py:341-356).  The reference runs one prefill per request with no such
 * split (prefill.py:69-72, slab_attention.py:376-476): this only changes how the work
 * is spread over the chip.  oscar_attn_prefill_v1 splits when workspace_bytes is at
 * least this size (and the workspace 16-byte aligned), else runs one workgroup per query
 * tile.  Returns -22 for invalid arguments. */
int64_t oscar_prefill_workspace_bytes_v2(int64_t history, int64_t num_tokens, int64_t num_q_heads,
                                         int64_t num_kv_heads, int64_t head_dim);

/* The split plan oscar_attn_prefill_v1 uses for these sizes (no counterpart in the
 * reference; for tests and callers sizing their own workspace): out[0..5] = chunks of the
 * heaviest tile (0: no split), key tiles (32 keys) per chunk, query tiles, first query tile
 * with two chunks, workgroups per KV head, partial slots per KV head; out[6 + c], c <=
 * chunks = first workgroup of chunk class c.  Needs cap >= 6 + 33.  Returns 0 or -22. */
int oscar_prefill_plan_v1(int64_t history, int64_t num_tokens, int64_t num_q_heads, int64_t num_kv_heads,
                          int32_t* out, int32_t cap);

/* ---- native decode step ------------------------------------------------------
 * One call per decode-shaped forward of the impl (backend.py:249-393 for batches whose
 * requests all have history: decode, MTP verification, cache-only decode, and cached
 * chunks of up to 16384 rows per KV head, which the plan cuts into 32-row sub-requests).  The call classifies the batch from the host metadata, builds
 * the split-K plan on the host, stages every integer array the kernels read through
 * the context's pinned ring in ONE host-to-device copy, and enqueues the store (or the
 * query rotation when there are no new tokens), the split-K decode and merge, and the
 * inverse rotation into `output` -- with no Python in between.  It returns
 * OSCAR_STEP_NOT_DECODE (nothing enqueued) when a request is history-free, its current
 * chunk has more than 16384 rows per KV head, Hq / Hk exceeds 32, the plan outgrows a
 * ring slot, or the requests do not tile [0, num_tokens): the caller then takes the
 * general path.
 *
 * The context holds a ring of pinned host and device metadata slots, reused once the
 * event recorded after the slot's last reader has completed; one per device, created
 * once (it allocates), used from any thread.  The step is eager-only: it builds the plan
 * on the host at every call, copies it from a ring slot that a later call rewrites, and
 * may wait on a ring event, so it must not be captured into a HIP graph (it returns -22
 * while `stream` is capturing).  Graph capture works with oscar_store_v1 and with
 * oscar_attn_decode_v1 / oscar_decode_write_v1 over a plan uploaded beforehand. */
typedef struct oscar_context_v1 oscar_context_v1;
int oscar_context_create_v1(int32_t device, oscar_context_v1** ctx);
int oscar_context_destroy_v1(oscar_context_v1* ctx);

#define OSCAR_STEP_NOT_DECODE 1

typedef struct oscar_step_args_v1 {
  const void* query;            /* [num_tokens, Hq, D] rows in q_dtype, token stride Hq * D */
  const void* key;              /* [num_tokens, Hk, D] or NULL (cache-only: no write) */
  const void* value;
  int64_t kv_stride_token;      /* elements */
  int64_t num_tokens;           /* num_actual_tokens */
  int64_t num_q_heads;
  int32_t q_dtype;              /* OSCAR_BF16 or OSCAR_F16 (key / value / output too) */
  int32_t stage_mode;           /* enum oscar_stage_mode, used when key != NULL */
  const int64_t* slot_mapping;  /* device [num_tokens] (key != NULL) */
  oscar_cache_v1 cache;
  const int32_t* block_table;   /* device [num_reqs, max_blocks] */
  int64_t block_table_stride;
  const oscar_staging_v1* staging; /* NULL: no FP32 window */
  int32_t sink_tokens_eff;
  int32_t recent_tokens;
  const float* rk;              /* [D, D] fp32, required */
  const float* rv;
  float k_clip_ratio;
  float v_clip_ratio;
  float scale;
  int32_t target_items;         /* split-K items (0: one per compute unit) */
  const int32_t* host_query_start_loc; /* host [num_reqs + 1] */
  const int32_t* host_seq_lens;        /* host [num_reqs] */
  int32_t num_reqs;
  int32_t reserved;
  void* output;                 /* [num_tokens, Hq, D] in q_dtype, token stride Hq * D */
  /* store scratch, as in oscar_store_args_v1 */
  int64_t* slot_claims;
  int64_t* seat_claims;
  int64_t* epoch_counter;
  void* store_workspace;
  int64_t store_workspace_bytes;
  uint32_t* arrivals;
  /* step workspace (rotated q / k / v, out_rot, lse, item partials), 256-byte aligned */
  void* workspace;
  int64_t workspace_bytes;
  int64_t workspace_needed;     /* out: bytes this call needed (set when it returns -28) */
  /* block_table geometry [rows, cols], checked on the host before anything is enqueued
   * (streaming_attention.py:48-53): rows < num_reqs -> -22 "Missing request block-table
   * rows"; a request with queries whose history (seq - its query count with key / value,
   * else seq) needs more than cols pages -> -22 "Block table cannot cover the history" */
  int64_t block_table_rows;
  int64_t block_table_cols;
} oscar_step_args_v1;

int64_t oscar_step_workspace_bytes_v1(int64_t num_tokens, int64_t num_q_heads, int64_t num_kv_heads,
                                      int64_t head_dim, int64_t num_items);
int oscar_decode_step_v1(oscar_context_v1* ctx, oscar_step_args_v1* args, void* stream);

const char* oscar_last_error(void);
int oscar_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* OSCAR_AMD_H */
