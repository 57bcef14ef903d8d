// attn_launch.hip -- host launchers (argument checks, parameter packing,
// variant dispatch) and the C ABI of include/pth_attn.h.
//
// Responsibilities follow the reference launcher (attn_launch.cu:63-236,
// attn_combine.cu:356-411, attn_capi.cu): every check names the field, the
// byte strides are copied as given, nothing is allocated, nothing is read
// back and nothing synchronises. The torch op (torch_op.cpp) and the C ABI
// both launch through launch_attention / launch_combine, so the op runs
// exactly the code the C-ABI tests exercise.

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

#include "attn_internal.h"

namespace pa {
namespace {

thread_local std::string g_last_error;

constexpr float kLog2e = 1.44269504088896340736f;
constexpr int64_t kVecAlign = 16;

bool aligned(const void* ptr, int64_t a) {
  return reinterpret_cast<uintptr_t>(ptr) % static_cast<uintptr_t>(a) == 0;
}

// A cache stream needs 4-byte alignment of its base and of every byte stride
// that multiplies a non-zero index (a size-1 dimension's stride never reaches
// an address). Reference cache_geometry.cuh:200-222 (the 4-byte floor).
bool stream_aligned(const PthAttnStream& s, const PthAttnArgs& a) {
  if (!aligned(s.data, 4)) return false;
  if (a.num_blocks > 1 && s.stride_block % 4 != 0) return false;
  if (a.block_size > 1 && s.stride_slot % 4 != 0) return false;
  if (a.num_kv_heads > 1 && s.stride_head % 4 != 0) return false;
  return true;
}

CacheStream cache_stream(const PthAttnStream& s) {
  return CacheStream{static_cast<const char*>(s.data), s.stride_block,
                     s.stride_slot, s.stride_head};
}

// Fills the cell view of the four streams when they share their strides and
// every per-lane offset the paged kernels form fits in 32 bits
// (cell_reach_fits: key < 16 of a 16-key group, any KV head, any stream,
// plus a head_size-byte row).
void set_cell_geometry(const PthAttnArgs& a, AttnParams& p) {
  p.cell = false;
  const PthAttnStream* st[4] = {&a.k_cache, &a.v_cache, &a.k_scale, &a.v_scale};
  const int64_t sb = st[0]->stride_block, ss = st[0]->stride_slot, sh = st[0]->stride_head;
  if (sb < 0 || ss < 0 || sh < 0) return;
  uintptr_t lo = reinterpret_cast<uintptr_t>(st[0]->data);
  for (int i = 0; i < 4; ++i) {
    if (st[i]->stride_block != sb || st[i]->stride_slot != ss || st[i]->stride_head != sh)
      return;
    lo = std::min(lo, reinterpret_cast<uintptr_t>(st[i]->data));
  }
  const uint64_t lim = uint64_t{1} << 32;
  uint64_t max_off = 0;
  for (int i = 0; i < 4; ++i) {
    const uint64_t off = reinterpret_cast<uintptr_t>(st[i]->data) - lo;
    if (off >= lim) return;
    p.cell_off[i] = static_cast<uint32_t>(off);
    max_off = std::max(max_off, off);
  }
  const uint64_t slot_reach = static_cast<uint64_t>(a.block_size) * static_cast<uint64_t>(ss);
  if (static_cast<uint64_t>(sb) >= lim || slot_reach >= lim ||
      !cell_reach_fits(static_cast<uint64_t>(ss), static_cast<uint64_t>(sh), a.num_kv_heads,
                       max_off, a.head_size))
    return;
  p.cell = true;
  p.cell_base = reinterpret_cast<const char*>(lo);
  p.cell_block = static_cast<uint32_t>(sb);
  p.cell_slot = static_cast<uint32_t>(ss);
  p.cell_head = static_cast<uint32_t>(sh);
}

}  // namespace

int32_t resident_workgroups() {
  // 8 waves per CU (2 per SIMD at <= 256 VGPRs) = one 8-wave work-group.
  constexpr int kMaxDevices = 64;
  static int32_t cached[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kMaxDevices && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 0;
  const int32_t wgs = cus;
  if (dev < kMaxDevices) cached[dev] = wgs;
  return wgs;
}

const char* last_error() { return g_last_error.c_str(); }
int32_t fail(int32_t code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
void clear_error() { g_last_error.clear(); }

// Launch constants of the split partition of an attention launch (they must
// be the same in the attention kernel, the combine and the unused-split
// fill): 16-row groups per row tile, groups of kGroupUnits KV-head units, and
// the attention grid (one work-group per CU).
void stream_fields(const PthAttnArgs& a, CombineParams& c) {
  const int32_t group = a.num_q_heads / a.num_kv_heads;
  const int32_t rows = a.bq * group;
  c.seq_lens = a.seq_lens;
  c.bq = a.bq;
  c.group = group;
  c.n_rg = (rows + kRowsPerWave - 1) / kRowsPerWave;
  c.gu = group_units(a.num_kv_heads * c.n_rg);
  c.n_hg = (a.num_kv_heads * c.n_rg + c.gu - 1) / c.gu;
  c.num_wg = resident_workgroups() * (kGroupUnits / c.gu);
  c.window = a.window;
  c.causal = a.causal;
}

int32_t launch_attention(const PthAttnArgs& a, int32_t loader,
                         hipStream_t stream, float* lse_out,
                         int64_t lse_stride_token, int64_t lse_stride_head,
                         bool fill_unused_splits) {
  clear_error();
  PA_REQUIRE(loader >= 0 && loader <= 2,
             "options.loader must be 0 (default), 1 (separate) or 2 (cell)");
  PA_REQUIRE(loader != 2,
             "options.loader = cell: the whole-cell loader is not built in "
             "this library (its kernels read the four streams separately)");
  PA_REQUIRE(a.q_dtype == PTH_ATTN_F16 || a.q_dtype == PTH_ATTN_BF16,
             "q_dtype must be PTH_ATTN_F16 or PTH_ATTN_BF16");
  PA_REQUIRE(a.out_dtype == PTH_ATTN_F32 || a.out_dtype == PTH_ATTN_F16 ||
                 a.out_dtype == PTH_ATTN_BF16,
             "out_dtype must be PTH_ATTN_F32, PTH_ATTN_F16 or PTH_ATTN_BF16");
  PA_REQUIRE(a.head_size == 64 || a.head_size == 128 || a.head_size == 256,
             "head_size must be 64, 128 or 256");
  PA_REQUIRE(a.head_size == 128 || (a.window == 0 && a.causal == 1),
             "sliding-window and non-causal attention need head size D = 128, got " +
                 std::to_string(a.head_size));
  PA_REQUIRE(a.num_kv_heads >= 1 && a.num_q_heads >= a.num_kv_heads &&
                 a.num_q_heads % a.num_kv_heads == 0,
             "num_q_heads must be a positive multiple of num_kv_heads");
  PA_REQUIRE(a.block_size >= 1, "block_size must be >= 1");
  PA_REQUIRE(a.num_blocks >= 1, "num_blocks must be >= 1");
  PA_REQUIRE(a.num_reqs >= 1, "num_reqs must be >= 1");
  PA_REQUIRE(a.num_tokens >= 1, "num_tokens must be >= 1");
  PA_REQUIRE(a.bq >= 1, "bq must be >= 1");
  PA_REQUIRE(a.num_splits >= 1, "num_splits must be >= 1");
  PA_REQUIRE(a.num_splits <= 65535, "num_splits must be <= 65535 (grid z)");
  PA_REQUIRE(a.num_q_tiles >= 0, "num_q_tiles must be >= 0");
  PA_REQUIRE(std::isfinite(a.softmax_scale) && a.softmax_scale > 0.0f,
             "softmax_scale must be finite and > 0");
  PA_REQUIRE(a.window >= 0, "window must be >= 0 (0 = none)");
  PA_REQUIRE(a.causal == 0 || a.causal == 1, "causal must be 0 or 1");
  PA_REQUIRE(a.q && a.k_cache.data && a.v_cache.data && a.k_scale.data &&
                 a.v_scale.data && a.block_table && a.seq_lens &&
                 a.query_start_loc,
             "q, the four cache streams, block_table, seq_lens and "
             "query_start_loc must be non-NULL");
  const int32_t group = a.num_q_heads / a.num_kv_heads;
  const int64_t rows = static_cast<int64_t>(a.bq) * group;
  PA_REQUIRE(rows <= 64, "bq * G = " + std::to_string(rows) +
                             " rows exceed one 64-row tile");
  PA_REQUIRE(aligned(a.q, kVecAlign) && a.q_stride_token % kVecAlign == 0 &&
                 a.q_stride_head % kVecAlign == 0,
             "q base and byte strides must be 16-B aligned");
  if (a.num_splits == 1) {
    PA_REQUIRE(a.out != nullptr, "out must be non-NULL when num_splits == 1");
    PA_REQUIRE(aligned(a.out, kVecAlign) &&
                   a.out_stride_token % kVecAlign == 0 &&
                   a.out_stride_head % kVecAlign == 0,
               "out base and byte strides must be 16-B aligned");
  } else {
    PA_REQUIRE(a.ws_o != nullptr && a.ws_lse != nullptr,
               "ws_o and ws_lse must be non-NULL when num_splits > 1");
    PA_REQUIRE(aligned(a.ws_o, kVecAlign) &&
                   a.ws_o_stride_split % kVecAlign == 0 &&
                   a.ws_o_stride_token % kVecAlign == 0 &&
                   a.ws_o_stride_head % kVecAlign == 0,
               "ws_o base and byte strides must be 16-B aligned");
    PA_REQUIRE(aligned(a.ws_lse, 4) && a.ws_lse_stride_split % 4 == 0 &&
                   a.ws_lse_stride_token % 4 == 0 &&
                   a.ws_lse_stride_head % 4 == 0,
               "ws_lse base and byte strides must be 4-B aligned");
  }
  const PthAttnStream* streams[4] = {&a.k_cache, &a.v_cache, &a.k_scale,
                                     &a.v_scale};
  for (int i = 0; i < 4; ++i) {
    PA_REQUIRE(stream_aligned(*streams[i], a),
               "cache stream " + std::to_string(i) +
                   " (K, V, k_scale, v_scale) is not 4-B aligned");
  }

  const int32_t n_rg = static_cast<int32_t>((rows + kRowsPerWave - 1) / kRowsPerWave);
  AttnParams p{};
  p.q = static_cast<const char*>(a.q);
  p.s_q_tok = a.q_stride_token;
  p.s_q_head = a.q_stride_head;
  p.out = static_cast<char*>(a.out);
  p.s_out_tok = a.out_stride_token;
  p.s_out_head = a.out_stride_head;
  p.ws_o = a.ws_o;
  p.s_wo_split = a.ws_o_stride_split;
  p.s_wo_tok = a.ws_o_stride_token;
  p.s_wo_head = a.ws_o_stride_head;
  p.ws_lse = a.ws_lse;
  p.s_wl_split = a.ws_lse_stride_split;
  p.s_wl_tok = a.ws_lse_stride_token;
  p.s_wl_head = a.ws_lse_stride_head;
  p.lse_out = lse_out;
  p.s_lo_tok = lse_stride_token;
  p.s_lo_head = lse_stride_head;
  p.k = cache_stream(a.k_cache);
  p.v = cache_stream(a.v_cache);
  p.ks = cache_stream(a.k_scale);
  p.vs = cache_stream(a.v_scale);
  set_cell_geometry(a, p);
  p.block_table = a.block_table;
  p.bt_stride = a.block_table_row_stride;
  p.seq_lens = a.seq_lens;
  p.qsl = a.query_start_loc;
  p.bs_div = Div32::make(static_cast<uint32_t>(a.block_size));
  p.g_div = Div32::make(static_cast<uint32_t>(group));
  p.bq_div = Div32::make(static_cast<uint32_t>(a.bq));
  p.rg_div = Div32::make(static_cast<uint32_t>(n_rg));
  p.num_reqs = a.num_reqs;
  p.n_hu = a.num_kv_heads * n_rg;
  p.gu = group_units(p.n_hu);
  p.n_hg = (p.n_hu + p.gu - 1) / p.gu;
  p.bq = a.bq;
  p.group = group;
  p.num_splits = a.num_splits;
  p.window = a.window;
  p.causal = a.causal;
  p.out_dtype = a.out_dtype;
  p.direct_single = fill_unused_splits ? 0 : 1;
  p.blk_tok = rows_block_tokens(group);
  p.num_kv_heads = a.num_kv_heads;
  p.scale_log2 = a.softmax_scale * kLog2e;
  p.page_rows = 0;
  if (p.cell && a.head_size == 128 && a.num_kv_heads == 8 && n_rg == 1 &&
      a.block_size % 16 == 0 && p.cell_head == 264 && p.cell_slot == 8 * 264) {
    bool inside = true;  // every stream of head h lies in bytes [264 h, 264 h + 264) of the row
    for (int i = 0; i < 4; ++i)
      inside = inside && p.cell_off[i] + (i < 2 ? 128u : 4u) <= 264u;
    p.page_rows = inside ? 1 : 0;
  }

  // Persistent grid. num_splits == 1: one wave per resident slot, but never
  // more waves than the unit table can hold (at most (T / bq + R) row tiles
  // x n_hu units). num_splits > 1: one work-group per CU, the partition's
  // work-group count.
  const int32_t wg_fill = resident_workgroups();
  PA_REQUIRE(wg_fill > 0, "cannot query the compute-unit count of the current device");
  int64_t wg = wg_fill;
  if (a.num_splits == 1) {
    const int64_t tile_bound =
        a.num_q_tiles > 0 ? a.num_q_tiles
                          : static_cast<int64_t>(a.num_tokens) / a.bq + a.num_reqs;
    const int64_t unit_bound = tile_bound * p.n_hu;
    PA_REQUIRE(unit_bound < 0x7fffffff, "the work table exceeds 2^31 - 1 units");
    const int64_t wg_need = (unit_bound + kGroupUnits - 1) / kGroupUnits;
    wg = wg_need < wg_fill ? wg_need : wg_fill;
  }
  const bool windowed = a.window > 0 || a.causal == 0;
  const bool paged16 = a.block_size % 16 == 0 && p.cell;
  // Row tiles of 64 rows (the planner's prefill and wide-verify plans) on a
  // single split: the row-block kernel, whose 8 waves share each key chunk
  // (one work-group per CU, never more than there are blocks).
  // Head sizes 64 and 256: the register-load kernel (any block size).
  const bool d128 = a.head_size == 128;
  const bool row_blocks = d128 && a.num_splits == 1 && paged16 && rows >= 64;
  hipError_t err;
  if (!d128) {
    const dim3 grid(static_cast<unsigned>(wg));
    err = launch_generic_kernel(p, grid, false, a.q_dtype == PTH_ATTN_F16, a.head_size, stream);
  } else if (row_blocks) {
    const int64_t blocks =
        (static_cast<int64_t>(a.num_tokens) / p.blk_tok + a.num_reqs) * a.num_kv_heads;
    PA_REQUIRE(blocks < 0x7fffffff, "the block table exceeds 2^31 - 1 blocks");
    const dim3 grid(static_cast<unsigned>(blocks < wg_fill ? blocks : wg_fill));
    err = launch_rows_kernel(p, grid, windowed, a.q_dtype == PTH_ATTN_F16, stream);
  } else {
    const dim3 grid(static_cast<unsigned>(wg));
    err = launch_fwd_kernel(p, grid, windowed, paged16, a.q_dtype == PTH_ATTN_F16, stream);
  }
  if (err != hipSuccess) {
    return fail(PTH_ATTN_ECUDA, std::string("attention launch (D=") +
                                    std::to_string(a.head_size) + ", rows=" +
                                    std::to_string(rows) + "): " +
                                    hipGetErrorString(err));
  }
  if (fill_unused_splits && a.num_splits > 1) {
    CombineParams f{};
    f.ws_lse = reinterpret_cast<const char*>(a.ws_lse);
    f.s_wl_split = a.ws_lse_stride_split;
    f.s_wl_tok = a.ws_lse_stride_token;
    f.s_wl_head = a.ws_lse_stride_head;
    f.qsl = a.query_start_loc;
    f.num_reqs = a.num_reqs;
    f.num_tokens = a.num_tokens;
    f.num_q_heads = a.num_q_heads;
    f.num_splits = a.num_splits;
    f.head_size = a.head_size;
    stream_fields(a, f);
    const hipError_t e2 = launch_fill_unused_splits(f, stream);
    if (e2 != hipSuccess)
      return fail(PTH_ATTN_ECUDA, std::string("unused-split fill launch: ") + hipGetErrorString(e2));
  }
  return PTH_ATTN_OK;
}

int32_t launch_combine(const PthAttnCombineArgs& c, hipStream_t stream,
                       float* lse_out, int64_t lse_stride_token,
                       int64_t lse_stride_head, const PthAttnArgs* split_source) {
  clear_error();
  PA_REQUIRE(c.head_size == 64 || c.head_size == 128 || c.head_size == 256,
             "head_size must be 64, 128 or 256");
  PA_REQUIRE(c.out_dtype == PTH_ATTN_F32 || c.out_dtype == PTH_ATTN_F16 ||
                 c.out_dtype == PTH_ATTN_BF16,
             "out_dtype must be PTH_ATTN_F32, PTH_ATTN_F16 or PTH_ATTN_BF16");
  PA_REQUIRE(c.num_splits >= 1, "num_splits must be >= 1");
  PA_REQUIRE(c.num_reqs >= 1, "num_reqs must be >= 1");
  PA_REQUIRE(c.num_tokens >= 1, "num_tokens must be >= 1");
  PA_REQUIRE(c.num_q_heads >= 1, "num_q_heads must be >= 1");
  PA_REQUIRE(c.ws_o && c.ws_lse && c.out && c.query_start_loc,
             "ws_o, ws_lse, out and query_start_loc must be non-NULL");
  // Each lane reads (and writes) D / 64 consecutive columns.
  const int64_t cols = c.head_size / 64;
  PA_REQUIRE(aligned(c.ws_o, 4 * cols) && c.ws_o_stride_split % (4 * cols) == 0 &&
                 c.ws_o_stride_token % (4 * cols) == 0 && c.ws_o_stride_head % (4 * cols) == 0,
             "ws_o base and byte strides must be aligned to D / 64 floats");
  PA_REQUIRE(aligned(c.ws_lse, 4) && c.ws_lse_stride_split % 4 == 0 &&
                 c.ws_lse_stride_token % 4 == 0 &&
                 c.ws_lse_stride_head % 4 == 0,
             "ws_lse base and byte strides must be 4-B aligned");
  const int64_t elem = (c.out_dtype == PTH_ATTN_F32 ? 4 : 2) * cols;
  PA_REQUIRE(aligned(c.out, elem) && c.out_stride_token % elem == 0 &&
                 c.out_stride_head % elem == 0,
             "out base and byte strides must be aligned to D / 64 elements");
  CombineParams p{};
  p.ws_o = reinterpret_cast<const char*>(c.ws_o);
  p.s_wo_split = c.ws_o_stride_split;
  p.s_wo_tok = c.ws_o_stride_token;
  p.s_wo_head = c.ws_o_stride_head;
  p.ws_lse = reinterpret_cast<const char*>(c.ws_lse);
  p.s_wl_split = c.ws_lse_stride_split;
  p.s_wl_tok = c.ws_lse_stride_token;
  p.s_wl_head = c.ws_lse_stride_head;
  p.out = static_cast<char*>(c.out);
  p.s_out_tok = c.out_stride_token;
  p.s_out_head = c.out_stride_head;
  p.out_dtype = c.out_dtype;
  p.lse_out = lse_out;
  p.s_lo_tok = lse_stride_token;
  p.s_lo_head = lse_stride_head;
  p.qsl = c.query_start_loc;
  p.num_reqs = c.num_reqs;
  p.num_tokens = c.num_tokens;
  p.num_q_heads = c.num_q_heads;
  p.num_splits = c.num_splits;
  p.head_size = c.head_size;
  if (split_source != nullptr) stream_fields(*split_source, p);
  const int64_t rows = static_cast<int64_t>(c.num_tokens) * c.num_q_heads;
  p.shared_rows = c.num_splits > 64 && rows < 4 * static_cast<int64_t>(resident_workgroups());
  const hipError_t err = launch_combine_kernel(p, stream);
  if (err != hipSuccess) {
    return fail(PTH_ATTN_ECUDA, std::string("combine launch: ") + hipGetErrorString(err));
  }
  return PTH_ATTN_OK;
}

}  // namespace pa

// ----------------------------------------------------------------- C ABI
namespace {
template <class T>
bool abi_matches(const T* a) {
  return a->abi_version == PTH_ATTN_ABI_VERSION &&
         a->struct_bytes == static_cast<int32_t>(sizeof(T));
}

int32_t check_args_abi(const PthAttnArgs* args) {
  PA_REQUIRE(args != nullptr, "args is NULL");
  PA_REQUIRE(args->abi_version == PTH_ATTN_ABI_VERSION,
             "abi_version " + std::to_string(args->abi_version) +
                 " != library ABI " + std::to_string(PTH_ATTN_ABI_VERSION));
  PA_REQUIRE(args->struct_bytes == static_cast<int32_t>(sizeof(PthAttnArgs)),
             "struct_bytes " + std::to_string(args->struct_bytes) +
                 " != sizeof(PthAttnArgs) " + std::to_string(sizeof(PthAttnArgs)));
  return PTH_ATTN_OK;
}

PthAttnCombineArgs combine_of(const PthAttnArgs& a) {
  PthAttnCombineArgs c{};
  c.abi_version = PTH_ATTN_ABI_VERSION;
  c.struct_bytes = static_cast<int32_t>(sizeof(PthAttnCombineArgs));
  c.ws_o = a.ws_o;
  c.ws_o_stride_split = a.ws_o_stride_split;
  c.ws_o_stride_token = a.ws_o_stride_token;
  c.ws_o_stride_head = a.ws_o_stride_head;
  c.ws_lse = a.ws_lse;
  c.ws_lse_stride_split = a.ws_lse_stride_split;
  c.ws_lse_stride_token = a.ws_lse_stride_token;
  c.ws_lse_stride_head = a.ws_lse_stride_head;
  c.out = a.out;
  c.out_dtype = a.out_dtype;
  c.out_stride_token = a.out_stride_token;
  c.out_stride_head = a.out_stride_head;
  c.query_start_loc = a.query_start_loc;
  c.num_reqs = a.num_reqs;
  c.num_tokens = a.num_tokens;
  c.num_q_heads = a.num_q_heads;
  c.head_size = a.head_size;
  c.num_splits = a.num_splits;
  return c;
}
// Scratch of pth_attn_attention_lse_noalloc: the split partials (ws_o, then
// ws_lse) of a launch live in this array instead of a caller's workspace.
// Every GPU the library runs on holds its own copy until the process ends.
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): each device's address is looked up once
// with hipGetSymbolAddress, with that device current, and kept per device.
// Nothing in it has to start at zero: a launch writes every partial slot and
// split-count marker its combine reads before the combine runs.
constexpr int64_t kScratchBytes = int64_t{64} << 20;
static __device__ __attribute__((aligned(256))) char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's address of `scratch` (looked up on the first call on
// that device).
int32_t scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pa::fail(PTH_ATTN_ECUDA, std::string("hipGetDevice: ") + hipGetErrorString(e));
  PA_REQUIRE(dev >= 0 && dev < kMaxScratchDevices,
             "device ordinal " + std::to_string(dev) + " is beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return pa::fail(PTH_ATTN_ECUDA, std::string("hipGetSymbolAddress(scratch): ") +
                                          hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PTH_ATTN_OK;
}

// Bytes of the dense partial layout of `a` in the scratch: ws_o
// [S, T, Hq, D] fp32 (256-byte aligned size), then ws_lse [S, T, Hq] fp32.
int64_t scratch_o_bytes(const PthAttnArgs& a) {
  const int64_t o = static_cast<int64_t>(a.num_splits) * a.num_tokens * a.num_q_heads *
                    a.head_size * 4;
  return (o + 255) / 256 * 256;
}
int64_t scratch_bytes(const PthAttnArgs& a) {
  return scratch_o_bytes(a) + static_cast<int64_t>(a.num_splits) * a.num_tokens * a.num_q_heads * 4;
}
}  // namespace

extern "C" {

int32_t pth_attn_abi_version(void) { return PTH_ATTN_ABI_VERSION; }
int32_t pth_attn_attn_args_bytes(void) { return static_cast<int32_t>(sizeof(PthAttnArgs)); }
int32_t pth_attn_combine_args_bytes(void) {
  return static_cast<int32_t>(sizeof(PthAttnCombineArgs));
}
int32_t pth_attn_options_bytes(void) { return static_cast<int32_t>(sizeof(PthAttnOptions)); }
int32_t pth_attn_has_cuda(void) { return 1; }
const char* pth_attn_last_error(void) { return pa::last_error(); }

int32_t pth_attn_tiling(int32_t head_size, int32_t bq, int32_t group,
                        int32_t* n_tile, int32_t* sub_tile, int32_t* wn) {
  pa::clear_error();
  PA_REQUIRE(head_size == 64 || head_size == 128 || head_size == 256,
             "head_size must be 64, 128 or 256");
  PA_REQUIRE(bq >= 1 && group >= 1, "bq and group must be >= 1");
  PA_REQUIRE(n_tile && sub_tile && wn, "output pointers must be non-NULL");
  PA_REQUIRE(static_cast<int64_t>(bq) * group <= 64, "bq * G exceeds 64 rows");
  *n_tile = pa::kTileTokens;
  *sub_tile = pa::kChunkTokens;
  *wn = (bq * group + pa::kRowsPerWave - 1) / pa::kRowsPerWave;
  return PTH_ATTN_OK;
}

int32_t pth_attn_attention_ex(const PthAttnArgs* args,
                              const PthAttnOptions* options, void* stream) {
  pa::clear_error();
  const int32_t rc = check_args_abi(args);
  if (rc != PTH_ATTN_OK) return rc;
  int32_t loader = 0;
  if (options != nullptr) {
    PA_REQUIRE(abi_matches(options), "options: abi_version/struct_bytes mismatch");
    loader = options->loader;
  }
  // A caller of this entry may combine all S splits itself
  // (pth_attn_combine), so the unused split slots get -inf.
  return pa::launch_attention(*args, loader, static_cast<hipStream_t>(stream),
                              nullptr, 0, 0, /*fill_unused_splits=*/true);
}

int32_t pth_attn_attention(const PthAttnArgs* args, void* stream) {
  return pth_attn_attention_ex(args, nullptr, stream);
}

int32_t pth_attn_attention_kernel(const PthAttnArgs* args, void* stream) {
  pa::clear_error();
  const int32_t rc = check_args_abi(args);
  if (rc != PTH_ATTN_OK) return rc;
  return pa::launch_attention(*args, 0, static_cast<hipStream_t>(stream), nullptr, 0, 0,
                              /*fill_unused_splits=*/false);
}

int32_t pth_attn_combine_kernel(const PthAttnArgs* args, void* stream) {
  pa::clear_error();
  const int32_t rc = check_args_abi(args);
  if (rc != PTH_ATTN_OK) return rc;
  PA_REQUIRE(args->num_splits > 1, "num_splits must be > 1 (a single split has no combine)");
  PA_REQUIRE(args->out != nullptr, "out must be non-NULL");
  return pa::launch_combine(combine_of(*args), static_cast<hipStream_t>(stream), nullptr, 0, 0,
                            args);
}

int32_t pth_attn_combine(const PthAttnCombineArgs* args, void* stream) {
  pa::clear_error();
  PA_REQUIRE(args != nullptr, "args is NULL");
  PA_REQUIRE(abi_matches(args), "abi_version/struct_bytes mismatch");
  return pa::launch_combine(*args, static_cast<hipStream_t>(stream), nullptr, 0, 0, nullptr);
}

int32_t pth_attn_attention_lse(const PthAttnArgs* args, float* lse,
                               int64_t lse_stride_token,
                               int64_t lse_stride_head, void* stream) {
  pa::clear_error();
  int32_t rc = check_args_abi(args);
  if (rc != PTH_ATTN_OK) return rc;
  PA_REQUIRE(lse != nullptr, "lse must be non-NULL");
  PA_REQUIRE(args->out != nullptr, "out must be non-NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  rc = pa::launch_attention(*args, 0, st, lse, lse_stride_token, lse_stride_head,
                            /*fill_unused_splits=*/false);
  if (rc != PTH_ATTN_OK || args->num_splits == 1) return rc;
  return pa::launch_combine(combine_of(*args), st, lse, lse_stride_token, lse_stride_head,
                            args);
}

int32_t pth_attn_attention_lse_noalloc(const PthAttnArgs* args, float* lse,
                                       int64_t lse_stride_token, int64_t lse_stride_head,
                                       void* stream) {
  pa::clear_error();
  int32_t rc = check_args_abi(args);
  if (rc != PTH_ATTN_OK) return rc;
  PA_REQUIRE(args->out != nullptr, "out must be non-NULL");
  PthAttnArgs a = *args;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (a.num_splits > 1) {
    PA_REQUIRE(a.num_tokens >= 1 && a.num_q_heads >= 1 &&
                   (a.head_size == 64 || a.head_size == 128 || a.head_size == 256),
               "num_tokens, num_q_heads and head_size must be valid to size the scratch");
    const int64_t need = scratch_bytes(a);
    PA_REQUIRE(need <= kScratchBytes,
               "the split partials need " + std::to_string(need) +
                   " bytes (num_splits x num_tokens x num_q_heads x (head_size + 1) x 4); "
                   "the static scratch holds " + std::to_string(kScratchBytes) +
                   " bytes: lower num_splits or split the batch");
    void* base = nullptr;
    rc = scratch_address(&base);
    if (rc != PTH_ATTN_OK) return rc;
    char* b = static_cast<char*>(base);
    const int64_t hd = static_cast<int64_t>(a.head_size) * 4;
    a.ws_o = reinterpret_cast<float*>(b);
    a.ws_o_stride_head = hd;
    a.ws_o_stride_token = hd * a.num_q_heads;
    a.ws_o_stride_split = a.ws_o_stride_token * a.num_tokens;
    a.ws_lse = reinterpret_cast<float*>(b + scratch_o_bytes(a));
    a.ws_lse_stride_head = 4;
    a.ws_lse_stride_token = 4 * static_cast<int64_t>(a.num_q_heads);
    a.ws_lse_stride_split = a.ws_lse_stride_token * a.num_tokens;
  }
  rc = pa::launch_attention(a, 0, st, lse, lse_stride_token, lse_stride_head,
                            /*fill_unused_splits=*/false);
  if (rc != PTH_ATTN_OK || a.num_splits == 1) return rc;
  return pa::launch_combine(combine_of(a), st, lse, lse_stride_token, lse_stride_head, &a);
}

}  // extern "C"
