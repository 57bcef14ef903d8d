// torch_op.cpp -- the torch op pth_flash_attn::pth_flash_attn_fwd on ROCm.
//
// Drop-in for the reference op (csrc/pth_attn/torch_bindings.cpp:20-38,
// launch.cu:166-552): the same schema, the same argument checks in the same
// order with the same messages, registered for the CUDA key (HIP tensors on
// ROCm torch) and for the CPU key, where a valid call raises after the checks
// so that the checks are testable without a GPU. The one deliberate change
// is the device check: the reference requires compute capability 8.x, this
// library requires a gfx950 (MI355X) device.
//
// The op translates tensors into PthAttnArgs and calls the launchers of
// libpth_attn.so (pa::launch_attention / pa::launch_combine), the same code
// the C ABI runs. It allocates nothing, reads no device data on the host and
// never synchronises, so a call can be captured in a HIP graph.

#include <ATen/core/Tensor.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <hip/hip_runtime.h>
#include <torch/library.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "attn_internal.h"

namespace {

using at::Tensor;
using c10::ScalarType;

constexpr int64_t kRowsPerWave = 16;   // query rows per 16-row group (wm unit)
constexpr int64_t kMaxGroupSize = 64;  // one 64-row tile holds a whole group
constexpr int64_t kCacheAlign = 4;     // cache streams: 4-byte floor
constexpr int64_t kVectorAlign = 16;   // q, out, ws_o: 16-byte vectors

#define PFA_CHECK(cond, ...) TORCH_CHECK((cond), "pth_flash_attn_fwd: ", __VA_ARGS__)

const char* dtype_name(ScalarType t) {
  switch (t) {
    case ScalarType::BFloat16: return "bfloat16";
    case ScalarType::Half: return "float16";
    case ScalarType::Float: return "float32";
    case ScalarType::Char: return "int8";
    case ScalarType::Int: return "int32";
    case ScalarType::Long: return "int64";
    default: return "an unsupported dtype";
  }
}

void check_dtype(const Tensor& t, ScalarType want, const char* name) {
  PFA_CHECK(t.scalar_type() == want, name, " must be ", dtype_name(want), ", got ",
            dtype_name(t.scalar_type()));
}
void check_dim(const Tensor& t, int64_t want, const char* name) {
  PFA_CHECK(t.dim() == want, name, " must be ", want, "-D, got ", t.dim(), "-D");
}
void check_size(const Tensor& t, int64_t dim, int64_t want, const char* name,
                const char* what) {
  PFA_CHECK(t.size(dim) == want, name, ".size(", dim, ") must equal ", what, " = ", want,
            ", got ", t.size(dim));
}
void check_inner_stride_one(const Tensor& t, const char* name) {
  PFA_CHECK(t.stride(t.dim() - 1) == 1, name,
            " must have stride 1 in its last dimension, got ", t.stride(t.dim() - 1));
}
void check_same_device(const Tensor& t, const Tensor& ref, const char* name) {
  PFA_CHECK(t.device() == ref.device(), name, " must be on the same device as q");
}

// Largest reachable byte offset + one element, with overflow and negative
// strides rejected (reference ops.h:65-87).
bool view_extent_bytes(const Tensor& t, int64_t* extent) {
  const int64_t elem = static_cast<int64_t>(t.element_size());
  for (int64_t i = 0; i < t.dim(); ++i) {
    if (t.size(i) < 0 || t.stride(i) < 0) return false;
    if (t.size(i) == 0) {
      *extent = 0;
      return true;
    }
  }
  int64_t total = elem;
  for (int64_t i = 0; i < t.dim(); ++i) {
    int64_t term = 0;
    if (__builtin_mul_overflow(t.size(i) - 1, t.stride(i), &term) ||
        __builtin_mul_overflow(term, elem, &term) ||
        __builtin_add_overflow(total, term, &total))
      return false;
  }
  *extent = total;
  return true;
}

void check_int64_extent(const Tensor& t, const char* name) {
  int64_t extent = 0;
  PFA_CHECK(view_extent_bytes(t, &extent), name,
            " has negative strides or a byte extent that overflows int64");
}

void check_alignment(const Tensor& t, int64_t align, const char* name) {
  const auto addr = reinterpret_cast<uintptr_t>(t.data_ptr());
  PFA_CHECK(addr % static_cast<uintptr_t>(align) == 0, name, " data pointer must be ", align,
            "-byte aligned");
  const int64_t elem = static_cast<int64_t>(t.element_size());
  for (int64_t i = 0; i + 1 < t.dim(); ++i) {
    PFA_CHECK((t.stride(i) * elem) % align == 0, name, " byte stride of dim ", i, " (",
              t.stride(i) * elem, ") must be a multiple of ", align);
  }
}

// Metadata checks; the Python fake (ops.py) runs the same list with the same
// messages (reference launch.cu:166-310).
void check_metadata(const Tensor& out, const Tensor& q, const Tensor& k_cache,
                    const Tensor& v_cache, const Tensor& k_scale, const Tensor& v_scale,
                    const Tensor& block_table, const Tensor& seq_lens,
                    const Tensor& query_start_loc, int64_t max_query_len, int64_t wm,
                    int64_t num_splits, double softmax_scale, const Tensor& ws_o,
                    const Tensor& ws_lse, int64_t window, bool causal) {
  check_dim(q, 3, "q");
  PFA_CHECK(q.scalar_type() == ScalarType::BFloat16 || q.scalar_type() == ScalarType::Half,
            "q must be bfloat16 or float16, got ", dtype_name(q.scalar_type()));
  const int64_t T = q.size(0), Hq = q.size(1), D = q.size(2);
  PFA_CHECK(D == 64 || D == 128 || D == 256,
            "head size D = q.size(2) must be 64, 128 or 256, got ", D);
  check_inner_stride_one(q, "q");

  check_dim(out, 3, "out");
  check_dtype(out, q.scalar_type(), "out (same dtype as q)");
  check_size(out, 0, T, "out", "T");
  check_size(out, 1, Hq, "out", "Hq");
  check_size(out, 2, D, "out", "D");
  check_inner_stride_one(out, "out");

  check_dim(k_cache, 4, "k_cache");
  check_dim(v_cache, 4, "v_cache");
  check_dtype(k_cache, ScalarType::Char, "k_cache");
  check_dtype(v_cache, ScalarType::Char, "v_cache");
  const int64_t NB = k_cache.size(0), BS = k_cache.size(1), Hkv = k_cache.size(2);
  check_size(k_cache, 3, D, "k_cache", "D");
  check_size(v_cache, 0, NB, "v_cache", "NB");
  check_size(v_cache, 1, BS, "v_cache", "BS");
  check_size(v_cache, 2, Hkv, "v_cache", "Hkv");
  check_size(v_cache, 3, D, "v_cache", "D");
  check_inner_stride_one(k_cache, "k_cache");
  check_inner_stride_one(v_cache, "v_cache");

  check_dim(k_scale, 3, "k_scale");
  check_dim(v_scale, 3, "v_scale");
  check_dtype(k_scale, ScalarType::Float, "k_scale");
  check_dtype(v_scale, ScalarType::Float, "v_scale");
  check_size(k_scale, 0, NB, "k_scale", "NB");
  check_size(k_scale, 1, BS, "k_scale", "BS");
  check_size(k_scale, 2, Hkv, "k_scale", "Hkv");
  check_size(v_scale, 0, NB, "v_scale", "NB");
  check_size(v_scale, 1, BS, "v_scale", "BS");
  check_size(v_scale, 2, Hkv, "v_scale", "Hkv");

  PFA_CHECK(Hkv >= 1 && Hq % Hkv == 0, "Hq = ", Hq, " must be a positive multiple of Hkv = ",
            Hkv);
  const int64_t G = Hq / Hkv;
  PFA_CHECK(wm == 1 || wm == 2 || wm == 4, "wm must be 1, 2 or 4, got ", wm);
  PFA_CHECK(G <= kMaxGroupSize, "G = Hq/Hkv = ", G, " exceeds the supported maximum ",
            kMaxGroupSize);
  PFA_CHECK(G <= kRowsPerWave * wm, "G = Hq/Hkv = ", G, " must be <= 16*wm = ",
            kRowsPerWave * wm);

  check_dim(block_table, 2, "block_table");
  check_dim(seq_lens, 1, "seq_lens");
  check_dim(query_start_loc, 1, "query_start_loc");
  check_dtype(block_table, ScalarType::Int, "block_table");
  check_dtype(seq_lens, ScalarType::Int, "seq_lens");
  check_dtype(query_start_loc, ScalarType::Int, "query_start_loc");
  check_inner_stride_one(block_table, "block_table");
  check_inner_stride_one(seq_lens, "seq_lens");
  check_inner_stride_one(query_start_loc, "query_start_loc");
  const int64_t R = seq_lens.size(0);
  check_size(query_start_loc, 0, R + 1, "query_start_loc", "num_reqs + 1");
  PFA_CHECK(block_table.size(0) >= R, "block_table has ", block_table.size(0),
            " rows, fewer than num_reqs = ", R);

  PFA_CHECK(max_query_len >= 0 && max_query_len <= T, "max_query_len must be in [0, T = ", T,
            "], got ", max_query_len);
  PFA_CHECK(num_splits >= 1, "num_splits must be >= 1, got ", num_splits);
  PFA_CHECK(std::isfinite(softmax_scale) && softmax_scale > 0.0,
            "softmax_scale must be finite and > 0, got ", softmax_scale);
  PFA_CHECK(window >= 0, "window must be >= 0, got ", window);
  PFA_CHECK(!((window > 0 || !causal) && D != 128),
            "sliding-window and non-causal attention need head size D = 128, got ", D);

  check_same_device(out, q, "out");
  check_same_device(k_cache, q, "k_cache");
  check_same_device(v_cache, q, "v_cache");
  check_same_device(k_scale, q, "k_scale");
  check_same_device(v_scale, q, "v_scale");
  check_same_device(block_table, q, "block_table");
  check_same_device(seq_lens, q, "seq_lens");
  check_same_device(query_start_loc, q, "query_start_loc");

  if (num_splits > 1) {
    check_dim(ws_o, 4, "ws_o");
    check_dim(ws_lse, 3, "ws_lse");
    check_dtype(ws_o, ScalarType::Float, "ws_o");
    check_dtype(ws_lse, ScalarType::Float, "ws_lse");
    PFA_CHECK(ws_o.size(0) >= num_splits && ws_o.size(1) >= T,
              "ws_o must have size(0) >= num_splits = ", num_splits, " and size(1) >= T = ", T,
              ", got [", ws_o.size(0), ", ", ws_o.size(1), ", ...]");
    check_size(ws_o, 2, Hq, "ws_o", "Hq");
    check_size(ws_o, 3, D, "ws_o", "D");
    PFA_CHECK(ws_lse.size(0) >= num_splits && ws_lse.size(1) >= T,
              "ws_lse must have size(0) >= num_splits = ", num_splits, " and size(1) >= T = ",
              T, ", got [", ws_lse.size(0), ", ", ws_lse.size(1), ", ...]");
    check_size(ws_lse, 2, Hq, "ws_lse", "Hq");
    check_inner_stride_one(ws_o, "ws_o");
    check_inner_stride_one(ws_lse, "ws_lse");
    check_same_device(ws_o, q, "ws_o");
    check_same_device(ws_lse, q, "ws_lse");
  }
}

// Checks that need data pointers (reference launch.cu:315-346).
void check_addresses(const Tensor& out, const Tensor& q, const Tensor& k_cache,
                     const Tensor& v_cache, const Tensor& k_scale, const Tensor& v_scale,
                     const Tensor& block_table, const Tensor& seq_lens,
                     const Tensor& query_start_loc, int64_t num_splits, const Tensor& ws_o,
                     const Tensor& ws_lse) {
  check_int64_extent(out, "out");
  check_int64_extent(q, "q");
  check_int64_extent(k_cache, "k_cache");
  check_int64_extent(v_cache, "v_cache");
  check_int64_extent(k_scale, "k_scale");
  check_int64_extent(v_scale, "v_scale");
  check_int64_extent(block_table, "block_table");
  check_int64_extent(seq_lens, "seq_lens");
  check_int64_extent(query_start_loc, "query_start_loc");
  check_alignment(k_cache, kCacheAlign, "k_cache");
  check_alignment(v_cache, kCacheAlign, "v_cache");
  check_alignment(k_scale, kCacheAlign, "k_scale");
  check_alignment(v_scale, kCacheAlign, "v_scale");
  check_alignment(q, kVectorAlign, "q");
  check_alignment(out, kVectorAlign, "out");
  if (num_splits > 1) {
    PFA_CHECK(ws_o.data_ptr() != nullptr && ws_lse.data_ptr() != nullptr,
              "workspace (ws_o, ws_lse) must be allocated when num_splits > 1");
    check_int64_extent(ws_o, "ws_o");
    check_int64_extent(ws_lse, "ws_lse");
    check_alignment(ws_o, kVectorAlign, "ws_o");
  }
}

// The kernels are built for gfx950 only (the reference checks for compute
// capability 8.x here, launch.cu:350-361).
void check_device_arch(const Tensor& q) {
  hipDeviceProp_t prop;
  const hipError_t err = hipGetDeviceProperties(&prop, q.get_device());
  PFA_CHECK(err == hipSuccess, "cannot query the device properties: ", hipGetErrorString(err));
  PFA_CHECK(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0,
            "needs a gfx950 (MI355X) device, device is ", prop.gcnArchName);
}

int64_t wm_for_rows(int64_t rows) {
  int64_t wm = 1;
  while (wm < 4 && rows > kRowsPerWave * wm) wm *= 2;
  return wm;
}

// Query tokens per row tile: max_query_len when that keeps the planned wm,
// else the capacity floor(16 wm / G) (reference launch.cu:363-387).
int32_t tile_tokens(int64_t wm, int64_t group, int64_t max_query_len) {
  const int64_t capacity = kRowsPerWave * wm / group;
  if (max_query_len >= 1 && max_query_len < capacity &&
      wm_for_rows(max_query_len * group) == wm)
    return static_cast<int32_t>(max_query_len);
  return static_cast<int32_t>(capacity);
}

void check_wm_matches_rows(int64_t wm, int64_t group, int32_t bq) {
  const int64_t rows = static_cast<int64_t>(bq) * group;
  const int64_t derived = wm_for_rows(rows);
  PFA_CHECK(derived == wm, "wm = ", wm, " is not the tile height of G = ", group, " (rows ",
            rows, " need wm = ", derived, ")");
}

int32_t dtype_code(ScalarType t) {
  return t == ScalarType::Half ? PTH_ATTN_F16 : PTH_ATTN_BF16;
}
int64_t byte_stride(const Tensor& t, int64_t dim) {
  return t.stride(dim) * static_cast<int64_t>(t.element_size());
}
PthAttnStream stream_of(const Tensor& t) {
  PthAttnStream s{};
  s.data = t.data_ptr();
  s.stride_block = byte_stride(t, 0);
  s.stride_slot = byte_stride(t, 1);
  s.stride_head = byte_stride(t, 2);
  return s;
}

void launch_library(const Tensor& out, const Tensor& q, const Tensor& k_cache,
                    const Tensor& v_cache, const Tensor& k_scale, const Tensor& v_scale,
                    const Tensor& block_table, const Tensor& seq_lens,
                    const Tensor& query_start_loc, int64_t max_query_len, int64_t wm,
                    int64_t num_splits, double softmax_scale, const Tensor& ws_o,
                    const Tensor& ws_lse, int64_t window, bool causal) {
  const int64_t Hkv = k_cache.size(2);
  const int64_t group = q.size(1) / Hkv;
  const int32_t bq = tile_tokens(wm, group, max_query_len);
  check_wm_matches_rows(wm, group, bq);

  PthAttnArgs a{};
  a.abi_version = PTH_ATTN_ABI_VERSION;
  a.struct_bytes = static_cast<int32_t>(sizeof(PthAttnArgs));
  a.q = q.data_ptr();
  a.q_dtype = dtype_code(q.scalar_type());
  a.q_stride_token = byte_stride(q, 0);
  a.q_stride_head = byte_stride(q, 1);
  a.out = out.data_ptr();
  a.out_dtype = dtype_code(out.scalar_type());
  a.out_stride_token = byte_stride(out, 0);
  a.out_stride_head = byte_stride(out, 1);
  a.k_cache = stream_of(k_cache);
  a.v_cache = stream_of(v_cache);
  a.k_scale = stream_of(k_scale);
  a.v_scale = stream_of(v_scale);
  a.num_blocks = static_cast<int32_t>(k_cache.size(0));
  a.block_size = static_cast<int32_t>(k_cache.size(1));
  a.num_kv_heads = static_cast<int32_t>(Hkv);
  a.head_size = static_cast<int32_t>(q.size(2));
  a.block_table = static_cast<const int32_t*>(block_table.data_ptr());
  a.block_table_row_stride = block_table.stride(0);
  a.seq_lens = static_cast<const int32_t*>(seq_lens.data_ptr());
  a.query_start_loc = static_cast<const int32_t*>(query_start_loc.data_ptr());
  a.num_reqs = static_cast<int32_t>(seq_lens.size(0));
  a.num_tokens = static_cast<int32_t>(q.size(0));
  a.num_q_heads = static_cast<int32_t>(q.size(1));
  a.bq = bq;
  a.num_q_tiles = 0;
  a.num_splits = static_cast<int32_t>(num_splits);
  a.softmax_scale = static_cast<float>(softmax_scale);
  a.window = window > INT32_MAX ? INT32_MAX : static_cast<int32_t>(window);
  a.causal = causal ? 1 : 0;
  if (num_splits > 1) {
    a.ws_o = static_cast<float*>(ws_o.data_ptr());
    a.ws_o_stride_split = byte_stride(ws_o, 0);
    a.ws_o_stride_token = byte_stride(ws_o, 1);
    a.ws_o_stride_head = byte_stride(ws_o, 2);
    a.ws_lse = static_cast<float*>(ws_lse.data_ptr());
    a.ws_lse_stride_split = byte_stride(ws_lse, 0);
    a.ws_lse_stride_token = byte_stride(ws_lse, 1);
    a.ws_lse_stride_head = byte_stride(ws_lse, 2);
  }

  // ROCm torch reports HIP tensors as device type "cuda"; the masquerading
  // guard and stream accept that type.
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const hipStream_t stream =
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  // The combine below reads only the splits each request used.
  int32_t rc = pa::launch_attention(a, 0, stream, nullptr, 0, 0, /*fill_unused_splits=*/false);
  PFA_CHECK(rc == PTH_ATTN_OK, "attention launch: ", pa::last_error());
  if (num_splits == 1) return;
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
  rc = pa::launch_combine(c, stream, nullptr, 0, 0, &a);
  PFA_CHECK(rc == PTH_ATTN_OK, "combine launch: ", pa::last_error());
}

void pth_flash_attn_fwd(const Tensor& out, const Tensor& q, const Tensor& k_cache,
                        const Tensor& v_cache, const Tensor& k_scale, const Tensor& v_scale,
                        const Tensor& block_table, const Tensor& seq_lens,
                        const Tensor& query_start_loc, int64_t max_query_len, int64_t wm,
                        int64_t num_splits, double softmax_scale, const Tensor& ws_o,
                        const Tensor& ws_lse, int64_t window, bool causal) {
  check_metadata(out, q, k_cache, v_cache, k_scale, v_scale, block_table, seq_lens,
                 query_start_loc, max_query_len, wm, num_splits, softmax_scale, ws_o, ws_lse,
                 window, causal);
  check_addresses(out, q, k_cache, v_cache, k_scale, v_scale, block_table, seq_lens,
                  query_start_loc, num_splits, ws_o, ws_lse);
  PFA_CHECK(q.is_cuda(),
            "arguments are valid, but the op computes on CUDA tensors only (the CPU "
            "registration exists to test the argument checks)");
  check_device_arch(q);
  if (q.size(0) == 0 || seq_lens.size(0) == 0) return;
  launch_library(out, q, k_cache, v_cache, k_scale, v_scale, block_table, seq_lens,
                 query_start_loc, max_query_len, wm, num_splits, softmax_scale, ws_o, ws_lse,
                 window, causal);
}

#define PFW_CHECK(cond, ...) TORCH_CHECK((cond), "reshape_and_cache_int8: ", __VA_ARGS__)

// vLLM's int8_per_token_head cache write (no op of the reference: it uses
// vLLM's Triton writer, mirrored by python/pth_testing/reference.py:76-103):
// key / value [T, Hkv, D] (fp32, fp16 or bf16) into the four cache views of
// pth_flash_attn_fwd, token t at slot slot_mapping[t] (< 0: skipped).
void reshape_and_cache_int8(const Tensor& key, const Tensor& value, const Tensor& k_cache,
                            const Tensor& v_cache, const Tensor& k_scale,
                            const Tensor& v_scale, const Tensor& slot_mapping) {
  PFW_CHECK(key.dim() == 3 && value.dim() == 3, "key and value must be 3-D [T, Hkv, D]");
  PFW_CHECK(key.sizes() == value.sizes(), "key and value must have the same shape");
  PFW_CHECK(key.scalar_type() == value.scalar_type() &&
                (key.scalar_type() == at::kFloat || key.scalar_type() == at::kHalf ||
                 key.scalar_type() == at::kBFloat16),
            "key and value must both be float32, float16 or bfloat16");
  PFW_CHECK(key.stride(2) == 1 && value.stride(2) == 1,
            "key and value must have stride 1 in their last dimension");
  const int64_t T = key.size(0), Hkv = key.size(1), D = key.size(2);
  PFW_CHECK(D == 64 || D == 128 || D == 256, "head size must be 64, 128 or 256, got ", D);
  PFW_CHECK(k_cache.dim() == 4 && v_cache.dim() == 4 && k_cache.scalar_type() == at::kChar &&
                v_cache.scalar_type() == at::kChar,
            "k_cache and v_cache must be 4-D int8 [num_blocks, block_size, Hkv, D]");
  PFW_CHECK(k_cache.sizes() == v_cache.sizes() && k_cache.size(2) == Hkv && k_cache.size(3) == D,
            "k_cache and v_cache must be [num_blocks, block_size, ", Hkv, ", ", D, "]");
  PFW_CHECK(k_cache.stride(3) == 1 && v_cache.stride(3) == 1,
            "k_cache and v_cache must have stride 1 in their last dimension");
  PFW_CHECK(k_scale.dim() == 3 && v_scale.dim() == 3 && k_scale.scalar_type() == at::kFloat &&
                v_scale.scalar_type() == at::kFloat &&
                k_scale.sizes() == k_cache.sizes().slice(0, 3) &&
                v_scale.sizes() == k_cache.sizes().slice(0, 3),
            "k_scale and v_scale must be float32 [num_blocks, block_size, Hkv]");
  PFW_CHECK(slot_mapping.dim() == 1 && slot_mapping.size(0) == T &&
                slot_mapping.scalar_type() == at::kLong,
            "slot_mapping must be int64 [T]");
  const Tensor* all[] = {&value, &k_cache, &v_cache, &k_scale, &v_scale, &slot_mapping};
  for (const Tensor* t : all)
    PFW_CHECK(t->device() == key.device(), "all tensors must be on the device of key");
  PFW_CHECK(key.is_cuda(),
            "arguments are valid, but the op computes on CUDA tensors only (the CPU "
            "registration exists to test the argument checks)");
  if (T == 0) return;
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
  PthAttnWriteArgs a{};
  a.abi_version = PTH_ATTN_ABI_VERSION;
  a.struct_bytes = static_cast<int32_t>(sizeof(PthAttnWriteArgs));
  a.key = key.data_ptr();
  a.value = value.data_ptr();
  a.key_stride_token = byte_stride(key, 0);
  a.key_stride_head = byte_stride(key, 1);
  a.value_stride_token = byte_stride(value, 0);
  a.value_stride_head = byte_stride(value, 1);
  a.kv_dtype = key.scalar_type() == at::kFloat ? PTH_ATTN_F32
               : key.scalar_type() == at::kHalf ? PTH_ATTN_F16
                                                : PTH_ATTN_BF16;
  a.num_tokens = static_cast<int32_t>(T);
  a.num_kv_heads = static_cast<int32_t>(Hkv);
  a.head_size = static_cast<int32_t>(D);
  a.slot_mapping = slot_mapping.data_ptr<int64_t>();
  a.k_cache = stream_of(k_cache);
  a.v_cache = stream_of(v_cache);
  a.k_scale = stream_of(k_scale);
  a.v_scale = stream_of(v_scale);
  a.block_size = static_cast<int32_t>(k_cache.size(1));
  a.num_blocks = static_cast<int32_t>(k_cache.size(0));
  const hipStream_t stream =
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  const int32_t rc = pa::launch_write_kv(a, stream);
  PFW_CHECK(rc == PTH_ATTN_OK, pa::last_error());
}

}  // namespace

// Schema text identical to the reference's (torch_bindings.cpp:20-27,
// ops.py:50-56, docs/api.md:171-173).
TORCH_LIBRARY(pth_flash_attn, m) {
  m.def(
      "pth_flash_attn_fwd(Tensor! out, Tensor q, Tensor k_cache, "
      "Tensor v_cache, Tensor k_scale, Tensor v_scale, Tensor block_table, "
      "Tensor seq_lens, Tensor query_start_loc, int max_query_len, int wm, "
      "int num_splits, float softmax_scale, Tensor! ws_o, Tensor! ws_lse, "
      "int window=0, bool causal=True) -> ()");
  // The cache writer (no counterpart in the reference; see above).
  m.def(
      "reshape_and_cache_int8(Tensor key, Tensor value, Tensor! k_cache, Tensor! v_cache, "
      "Tensor! k_scale, Tensor! v_scale, Tensor slot_mapping) -> ()");
}

TORCH_LIBRARY_IMPL(pth_flash_attn, CUDA, m) {
  m.impl("pth_flash_attn_fwd", &pth_flash_attn_fwd);
  m.impl("reshape_and_cache_int8", &reshape_and_cache_int8);
}

// Validates, then raises: CPU tensors exist only to test the checks.
TORCH_LIBRARY_IMPL(pth_flash_attn, CPU, m) {
  m.impl("pth_flash_attn_fwd", &pth_flash_attn_fwd);
  m.impl("reshape_and_cache_int8", &reshape_and_cache_int8);
}
