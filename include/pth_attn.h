/*
 * pth_attn.h -- C ABI of the MI355X (gfx950) paged int8 attention library
 * libpth_attn.so.
 *
 * Every declaration here is the drop-in counterpart of an interface of the
 * reference (noon-at-cgn/pth-flash-attn); the citation after each item names
 * the reference file:line it replaces. Struct layouts, field meanings, status
 * codes and the ABI version are kept identical on purpose, so that a ctypes
 * mirror written for the reference drives this library unchanged.
 *
 * Conventions (reference csrc/pth_attn/attn_args.h:1-56):
 *  - every stride is in BYTES, except block_table_row_stride, which is in
 *    int32 ELEMENTS (as block_table.stride(0));
 *  - pointers are device pointers; nothing is allocated, nothing is read back
 *    to the host, no call synchronises;
 *  - abi_version / struct_bytes are checked at the C ABI (a stale ctypes
 *    mirror fails loudly instead of passing garbage).
 *
 * Semantics of an attention launch. Query token i of request r
 * (q_len = qsl[r+1] - qsl[r], L = seq_lens[r], both read on the device) sits
 * at KV position p = L - q_len + i (bottom-right alignment). Query head h
 * reads KV head h / G, G = num_q_heads / num_kv_heads. It sees the keys
 * [lo, hi] with lo = window > 0 ? max(0, p - window + 1) : 0 and
 * hi = causal ? p : (window > 0 ? min(L - 1, p + window - 1) : L - 1).
 * The result is softmax(softmax_scale * q.k_deq) v_deq with
 * k_deq = k_scale * k_cache and v_deq = v_scale * v_cache.
 *  - num_splits == 1: out[token, head, :] is written for every query token of
 *    every request, in out_dtype.
 *  - num_splits > 1: split s of a query row writes ws_o[s, token, head, :]
 *    (its softmax-normalised output, fp32) and ws_lse[s, token, head]
 *    (m + log2(l) in log2 units of the scaled scores). A split that sees no
 *    key of the row writes ws_lse = -inf and leaves ws_o unread by the
 *    combine. `out` is written by the combine (pth_attn_combine).
 *  - rows of tokens >= qsl[num_reqs] are never written.
 * Combine: M = max over live splits of lse_s; w_s = exp2(lse_s - M), splits
 * with lse_s = -inf are skipped before ws_o is read; out = sum_s w_s o_s /
 * sum_s w_s, summed in the fixed order s = 0..S-1 (deterministic).
 */
#ifndef PTH_ATTN_H_
#define PTH_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference: csrc/pth_attn/attn_args.h:62 */
#define PTH_ATTN_ABI_VERSION 2

/* Element types of q and out. Reference: attn_args.h:65-69 */
typedef enum PthAttnDtype {
  PTH_ATTN_F32 = 0,  /* out only */
  PTH_ATTN_F16 = 1,  /* q or out */
  PTH_ATTN_BF16 = 2, /* q or out */
} PthAttnDtype;

/* Status codes. Reference: attn_args.h:71-76 (ECUDA = a HIP runtime call or
 * the kernel launch failed; ENOCUDA is kept for the numbering and unused). */
typedef enum PthAttnStatus {
  PTH_ATTN_OK = 0,
  PTH_ATTN_EINVAL = -1,
  PTH_ATTN_ECUDA = -2,
  PTH_ATTN_ENOCUDA = -3,
} PthAttnStatus;

/* One cache stream: a view of logical shape [num_blocks, block_size,
 * num_kv_heads, row] (row = head_size int8 for K/V, one fp32 for a scale)
 * whose innermost row is contiguous. Reference: attn_args.h:81-86 */
typedef struct PthAttnStream {
  const void* data;     /* view.data_ptr() */
  int64_t stride_block; /* bytes between kernel blocks (pages) */
  int64_t stride_slot;  /* bytes between slots of one block */
  int64_t stride_head;  /* bytes between KV heads of one slot */
} PthAttnStream;

/* Launch arguments of the attention kernel. Reference: attn_args.h:88-144 */
typedef struct PthAttnArgs {
  int32_t abi_version;  /* = PTH_ATTN_ABI_VERSION */
  int32_t struct_bytes; /* = sizeof(PthAttnArgs) as compiled by the caller */

  const void* q; /* [num_tokens, num_q_heads, head_size] */
  int32_t q_dtype; /* PTH_ATTN_F16 or PTH_ATTN_BF16 */
  int64_t q_stride_token;
  int64_t q_stride_head;

  void* out; /* [num_tokens, num_q_heads, head_size] (num_splits == 1) */
  int32_t out_dtype; /* PTH_ATTN_F32, PTH_ATTN_F16 or PTH_ATTN_BF16 */
  int64_t out_stride_token;
  int64_t out_stride_head;

  PthAttnStream k_cache; /* int8 rows of head_size bytes */
  PthAttnStream v_cache; /* int8 rows of head_size bytes */
  PthAttnStream k_scale; /* one fp32 per (block, slot, head) */
  PthAttnStream v_scale; /* one fp32 per (block, slot, head) */
  int32_t num_blocks;
  int32_t block_size; /* tokens per kernel block, >= 1 */
  int32_t num_kv_heads;
  int32_t head_size; /* D; this library computes D = 128 */

  const int32_t* block_table;     /* [>= num_reqs, *] kernel-block ids */
  int64_t block_table_row_stride; /* ELEMENTS between rows */
  const int32_t* seq_lens;        /* [num_reqs] KV length incl. new tokens */
  const int32_t* query_start_loc; /* [num_reqs + 1], starts at 0 */

  int32_t num_reqs;
  int32_t num_tokens;  /* rows of q/out/workspace (may exceed qsl[R]) */
  int32_t num_q_heads; /* multiple of num_kv_heads */
  int32_t bq;          /* query tokens per row tile, >= 1 */
  int32_t num_q_tiles; /* grid x; 0 = num_tokens / bq + num_reqs */
  int32_t num_splits;  /* S >= 1 */
  float softmax_scale; /* multiplies q.k before the softmax, > 0 */

  float* ws_o; /* [>= S, >= num_tokens, num_q_heads, head_size] fp32 */
  int64_t ws_o_stride_split;
  int64_t ws_o_stride_token;
  int64_t ws_o_stride_head;
  float* ws_lse; /* [>= S, >= num_tokens, num_q_heads] fp32 */
  int64_t ws_lse_stride_split;
  int64_t ws_lse_stride_token;
  int64_t ws_lse_stride_head;

  int32_t window; /* 0 = none, else the sliding window in tokens */
  int32_t causal; /* 1 = bottom-right causal, 0 = non-causal */
} PthAttnArgs;

/* Launch arguments of the split combine. Reference: attn_args.h:146-171 */
typedef struct PthAttnCombineArgs {
  int32_t abi_version;
  int32_t struct_bytes;

  const float* ws_o;
  int64_t ws_o_stride_split;
  int64_t ws_o_stride_token;
  int64_t ws_o_stride_head;
  const float* ws_lse;
  int64_t ws_lse_stride_split;
  int64_t ws_lse_stride_token;
  int64_t ws_lse_stride_head;

  void* out;
  int32_t out_dtype;
  int64_t out_stride_token;
  int64_t out_stride_head;

  const int32_t* query_start_loc; /* rows >= qsl[num_reqs] are skipped */
  int32_t num_reqs;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t head_size;
  int32_t num_splits;
} PthAttnCombineArgs;

/* Arguments of the int8 cache writer (pth_attn_write_kv). No counterpart in
 * the reference's ABI: the reference relies on vLLM's Triton writer
 * triton_reshape_and_cache_flash_per_token_head_quant (vLLM 0.31.0; its call
 * site and mirror: python/pth_testing/reference.py:76-103, 301-307), which
 * is not available on ROCm here. Token t of key/value goes to slot
 * slot_mapping[t] of the cache (page slot / block_size, in-page slot
 * slot % block_size); a negative slot skips the token. The cache views are
 * the four of PthAttnArgs (byte strides; the vLLM cell shares them). */
typedef struct PthAttnWriteArgs {
  int32_t abi_version;  /* = PTH_ATTN_ABI_VERSION */
  int32_t struct_bytes; /* = sizeof(PthAttnWriteArgs) */

  const void* key;   /* [num_tokens, num_kv_heads, head_size] */
  const void* value; /* [num_tokens, num_kv_heads, head_size] */
  int64_t key_stride_token; /* bytes */
  int64_t key_stride_head;
  int64_t value_stride_token;
  int64_t value_stride_head;
  int32_t kv_dtype; /* PTH_ATTN_F32, PTH_ATTN_F16 or PTH_ATTN_BF16 */
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t head_size; /* 64, 128 or 256 */
  const int64_t* slot_mapping; /* [num_tokens] */

  PthAttnStream k_cache; /* int8 [num_blocks, block_size, num_kv_heads, head_size] */
  PthAttnStream v_cache;
  PthAttnStream k_scale; /* fp32 [num_blocks, block_size, num_kv_heads] */
  PthAttnStream v_scale;
  int32_t block_size;
  int32_t num_blocks;
} PthAttnWriteArgs;

/* Loader choice of pth_attn_attention_ex. Reference: attn_capi.h:32-39.
 * loader: 0 = default, 1 = separate streams (the only loader of this
 * library; 0 and 1 are the same), 2 = whole cell (not built: EINVAL). */
typedef struct PthAttnOptions {
  int32_t abi_version;
  int32_t struct_bytes;
  int32_t loader;
} PthAttnOptions;

/* Library identity. Reference: attn_capi.h:80-83 */
int32_t pth_attn_abi_version(void);
int32_t pth_attn_attn_args_bytes(void);
int32_t pth_attn_combine_args_bytes(void);
int32_t pth_attn_options_bytes(void);
/* sizeof(PthAttnWriteArgs). No counterpart in the reference (see above). */
int32_t pth_attn_write_args_bytes(void);
/* 1: the library holds GPU kernels (always). Reference: attn_capi.h:86 */
int32_t pth_attn_has_cuda(void);
/* Message of the calling thread's last failure ("" after a success).
 * Reference: attn_capi.h:87, attn_launch.h:46-56 */
const char* pth_attn_last_error(void);

/* Tiling of the kernel chosen for (head_size, bq, group): *n_tile = KV tokens
 * per tile (64), *sub_tile = KV tokens per softmax step (32), *wn = query-row
 * groups of 16 per row tile. Reference: attn_capi.h:89-93 */
int32_t pth_attn_tiling(int32_t head_size, int32_t bq, int32_t group,
                        int32_t* n_tile, int32_t* sub_tile, int32_t* wn);

/* Enqueue on `stream` (a hipStream_t; NULL = the null stream), no sync.
 * Reference: attn_capi.h:96-99, attn_launch.h:46-48 */
int32_t pth_attn_attention(const PthAttnArgs* args, void* stream);
int32_t pth_attn_attention_ex(const PthAttnArgs* args,
                              const PthAttnOptions* options, void* stream);
int32_t pth_attn_combine(const PthAttnCombineArgs* args, void* stream);

/* Test entry: the attention launch of `args` followed, when
 * num_splits > 1, by the combine into args->out, and the final
 * natural-log log-sum-exp of every real query row written to
 * lse[token * lse_stride_token + head * lse_stride_head] (byte strides,
 * fp32). The op's schema carries no LSE; this entry exposes it for parity
 * tests without changing the schema. No counterpart in the reference's
 * ABI (the reference tests read log2-LSE partials instead, attn_args.h:38-44). */
int32_t pth_attn_attention_lse(const PthAttnArgs* args, float* lse,
                               int64_t lse_stride_token,
                               int64_t lse_stride_head, void* stream);

/* Benchmark entry: the attention kernel of `args` exactly as the torch op
 * launches it before its combine (rows whose keys form a single split are
 * written to args->out, the others to the split partials; the unused split
 * slots are not filled). With the combine of pth_attn_attention_lse this is
 * the op's layer call. No counterpart in the reference's ABI. */
int32_t pth_attn_attention_kernel(const PthAttnArgs* args, void* stream);

/* Benchmark entry: the split combine exactly as the torch op launches it
 * after pth_attn_attention_kernel of the same `args` (num_splits > 1): it
 * reads only the splits each row has and skips rows the attention kernel
 * wrote to args->out itself. Timing it alone separates the two kernels of a
 * layer call. No counterpart in the reference's ABI. */
int32_t pth_attn_combine_kernel(const PthAttnArgs* args, void* stream);

/* pth_attn_attention_lse with no allocation and no workspace argument: the
 * split partials live in a static device array of the library (64 MiB per
 * GPU, reserved when the library's code object loads onto a device, for every
 * user of the library whether or not it calls this entry, and held until the
 * process ends; its address is looked up on the first call) instead
 * of args->ws_o / args->ws_lse, which are ignored. lse may be NULL (then
 * this is the op's layer call: attention + combine into args->out). Rejects
 * with EINVAL, before any launch, a batch whose partials need more than the
 * array: num_splits x num_tokens x num_q_heads x (head_size + 1) x 4 bytes
 * (the ws_o part rounded up to 256) must be <= 64 MiB. Calls that overlap on
 * one GPU (two streams, two threads) share the array and race; serialise
 * them. No counterpart in the reference: it is for callers that cannot
 * allocate (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int32_t pth_attn_attention_lse_noalloc(const PthAttnArgs* args, float* lse,
                                       int64_t lse_stride_token,
                                       int64_t lse_stride_head, void* stream);

/* The int8 per-token-head cache writer: per (token, KV head), the fp32
 * absmax scale max(absmax / 127, 1e-6) and int8 = trunc(clamp(x * (1 /
 * scale) +- 0.5, -128, 127)), step for step as vLLM's writer (the reference's
 * mirror: python/pth_testing/reference.py:76-103), into the cache cells.
 * Enqueued on `stream`, no sync. No counterpart in the reference's ABI. */
int32_t pth_attn_write_kv(const PthAttnWriteArgs* args, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PTH_ATTN_H_ */
