// attn_internal.h -- device-side launch parameters and the host launchers of
// libpth_attn.so (not part of the C ABI; include/pth_attn.h is).

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "attn_geometry.h"
#include "pth_attn.h"

namespace pa {

// One cache stream as the kernels read it: byte strides of [NB, BS, Hkv].
struct CacheStream {
  const char* base;
  int64_t s_block;
  int64_t s_slot;
  int64_t s_head;
};

// Everything one attention launch reads; passed by value as the kernel
// argument. Built by launch_attention from PthAttnArgs.
struct AttnParams {
  const char* q;
  int64_t s_q_tok, s_q_head;
  char* out;
  int64_t s_out_tok, s_out_head;
  float* ws_o;
  int64_t s_wo_split, s_wo_tok, s_wo_head;
  float* ws_lse;
  int64_t s_wl_split, s_wl_tok, s_wl_head;
  float* lse_out;  // optional natural-log LSE of every row (S == 1 only)
  int64_t s_lo_tok, s_lo_head;
  CacheStream k, v, ks, vs;
  // The same four streams as one array of cells, for the paged kernel: one
  // base, common byte strides, and each stream's byte offset within a cell
  // (K, V, k_scale, v_scale). Set when the streams share their strides (the
  // vLLM cache: four views of one buffer); `cell` is false otherwise.
  bool cell;
  const char* cell_base;
  uint32_t cell_block, cell_slot, cell_head;
  uint32_t cell_off[4];
  const int32_t* block_table;
  int64_t bt_stride;  // elements
  const int32_t* seq_lens;
  const int32_t* qsl;
  Div32 bs_div;  // block size
  Div32 g_div;   // GQA group
  Div32 bq_div;  // query tokens per row tile
  Div32 rg_div;  // 16-row groups per row tile
  int32_t num_reqs;
  int32_t n_hu;  // KV-head units per row tile: num_kv_heads * row groups
  int32_t gu;    // KV-head units per stream group: group_units(n_hu)
  int32_t n_hg;  // stream groups per row tile: ceil(n_hu / gu)
  int32_t bq;    // query tokens per row tile
  int32_t group;
  int32_t num_splits;
  int32_t window;
  int32_t causal;
  int32_t out_dtype;
  // num_splits > 1: a row whose stream has a single split is written to out
  // (and lse_out) by the attention kernel itself, and the combine skips it.
  // Off when the caller combines all num_splits splits itself.
  int32_t direct_single;
  // Row-block kernel (attn_rows.hip): query tokens per block and KV heads.
  int32_t blk_tok;
  int32_t num_kv_heads;
  float scale_log2;  // softmax_scale * log2(e)
  // The page-row kernel applies (attn_staged.hip): the cell view is vLLM's
  // NHD cell of 8 KV heads (264-byte cells, 2112-byte slot rows), pages of a
  // multiple of 16 keys, and a work-group's 8 waves are the 8 KV heads.
  int32_t page_rows;
};

struct CombineParams {
  const char* ws_o;
  int64_t s_wo_split, s_wo_tok, s_wo_head;
  const char* ws_lse;
  int64_t s_wl_split, s_wl_tok, s_wl_head;
  char* out;
  int64_t s_out_tok, s_out_head;
  int32_t out_dtype;
  float* lse_out;  // optional natural-log LSE
  int64_t s_lo_tok, s_lo_head;
  const int32_t* qsl;
  int32_t num_reqs;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t num_splits;
  int32_t head_size;  // 64, 128 or 256
  // When seq_lens is non-NULL the combine reads only the splits the
  // attention kernel wrote for the row (the stream partition of
  // attn_geometry.h for these lengths and launch constants) and skips rows
  // with a single split, which the attention kernel wrote to out itself;
  // otherwise it reads all num_splits for every row.
  const int32_t* seq_lens;
  int32_t bq;
  int32_t group;
  int32_t n_rg;
  int32_t gu;      // KV-head units per stream group
  int32_t n_hg;
  int32_t num_wg;  // partition work-groups: attention work-groups x kGroupUnits / gu
  int32_t window;
  int32_t causal;
  // A work-group per row (rows with many splits are merged by 4 waves)
  // instead of a wave per row: set when the launch may have more than 64
  // splits per row and has few rows.
  int32_t shared_rows;
};

// Host launchers. They check their arguments, enqueue on `stream`, allocate
// nothing and never synchronise. Return PTH_ATTN_OK, EINVAL or ECUDA; the
// message of a failure is last_error() on the calling thread.
// fill_unused_splits: also write -inf into the split slots [live, S) that
// no request uses (needed when the caller combines all S splits itself; the
// combine launched with split_source reads only the live ones).
int32_t launch_attention(const PthAttnArgs& a, int32_t loader,
                         hipStream_t stream, float* lse_out,
                         int64_t lse_stride_token, int64_t lse_stride_head,
                         bool fill_unused_splits);
int32_t launch_combine(const PthAttnCombineArgs& c, hipStream_t stream,
                       float* lse_out, int64_t lse_stride_token,
                       int64_t lse_stride_head, const PthAttnArgs* split_source);

// Per-variant kernel launches (attn_fwd.hip, attn_combine.hip).
// Work-groups (of kGroupUnits waves) that fill the device once: one per CU.
int32_t resident_workgroups();
hipError_t launch_fwd_kernel(const AttnParams& p, dim3 grid, bool windowed,
                             bool paged16, bool q_f16, hipStream_t stream);
// The register-load kernel for any block size and cache strides, head size
// 64, 128 or 256 (attn_generic.hip); windowed / non-causal at 128 only.
hipError_t launch_staged_kernel(const AttnParams& p, dim3 grid, bool windowed, bool q_f16,
                                hipStream_t stream);
hipError_t launch_generic_kernel(const AttnParams& p, dim3 grid, bool windowed, bool q_f16,
                                 int head_size, hipStream_t stream);
// The row-block kernel (num_splits == 1, paged cell caches) and the query
// tokens of one of its blocks for GQA group `group`.
hipError_t launch_rows_kernel(const AttnParams& p, dim3 grid, bool windowed, bool q_f16,
                              hipStream_t stream);
int32_t rows_block_tokens(int32_t group);
hipError_t launch_combine_kernel(const CombineParams& c, hipStream_t stream);
hipError_t launch_fill_unused_splits(const CombineParams& c, hipStream_t stream);

// The int8 cache writer (attn_writer.hip).
int32_t launch_write_kv(const PthAttnWriteArgs& a, hipStream_t stream);

const char* last_error();
int32_t fail(int32_t code, const std::string& msg);
void clear_error();

}  // namespace pa

#define PA_REQUIRE(cond, msg)                                   \
  do {                                                          \
    if (!(cond)) return ::pa::fail(PTH_ATTN_EINVAL, (msg));     \
  } while (0)
