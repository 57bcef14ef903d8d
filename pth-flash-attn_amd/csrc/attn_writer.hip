// attn_writer.hip -- the gfx950 int8 per-token-head cache writer: vLLM's
// reshape_and_cache for the int8_per_token_head cache (the reference relies
// on vLLM's Triton writer, mirrored by python/pth_testing/reference.py:76-103;
// no counterpart in the reference's ABI).
//
// One wave per (token, KV head): the K row and the V row of D values each
// get their fp32 absmax, scale = max(absmax / 127, 1e-6), inverse 1 / scale
// (both correctly rounded fp32 divisions), and q = trunc(clamp(x * inv +-
// 0.5, -128, 127)) with every step a separate fp32 operation (contraction
// off), so the bytes equal the writer's. Lane l quantises the D / 64
// consecutive values [l D / 64, (l + 1) D / 64) of each row.

#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "attn_internal.h"

namespace pa {
namespace {

struct WriteParams {
  const char* key;
  const char* value;
  int64_t s_k_tok, s_k_head, s_v_tok, s_v_head;
  int32_t kv_dtype;
  int32_t num_tokens;
  int32_t num_kv_heads;
  const int64_t* slot_mapping;
  CacheStream k, v, ks, vs;
  int32_t block_size;
  int64_t num_slots;  // num_blocks * block_size
};

__device__ __forceinline__ float load_elem(const char* p, int32_t dtype) {
  if (dtype == PTH_ATTN_F32) return *reinterpret_cast<const float*>(p);
  if (dtype == PTH_ATTN_F16) return static_cast<float>(*reinterpret_cast<const _Float16*>(p));
  return static_cast<float>(*reinterpret_cast<const __bf16*>(p));
}

__device__ __forceinline__ float wave_absmax(float x) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) x = fmaxf(x, __shfl_xor(x, d));
  return x;
}

// One row of D values (lane's NC at x) -> int8 at dst, scale at sdst.
template <int NC>
__device__ __forceinline__ void quantize_row(const float (&x)[NC], char* dst, float* sdst,
                                             int lane) {
#pragma clang fp contract(off)
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) a = fmaxf(a, fabsf(x[i]));
  const float amax = wave_absmax(a);
  float s = amax / 127.0f;
  if (!(s >= 1e-6f)) s = 1e-6f;
  const float inv = 1.0f / s;
  int8_t q[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float v = x[i] * inv;
    v = v >= 0.0f ? v + 0.5f : v - 0.5f;
    v = v < -128.0f ? -128.0f : v;
    v = v > 127.0f ? 127.0f : v;
    q[i] = static_cast<int8_t>(v);  // truncates toward zero
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) dst[NC * lane + i] = static_cast<char>(q[i]);
  if (lane == 0) *sdst = s;
}

template <int D>
__global__ __launch_bounds__(256) void write_kv_int8(const WriteParams w) {
  constexpr int NC = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t tok = item / w.num_kv_heads;
  const int head = static_cast<int>(item - tok * w.num_kv_heads);
  if (tok >= w.num_tokens) return;
  const int64_t slot = w.slot_mapping[tok];
  if (slot < 0 || slot >= w.num_slots) return;  // padding token (or out of the cache)
  const int64_t page = slot / w.block_size;
  const int64_t in_page = slot - page * w.block_size;
  float xk[NC], xv[NC];
  const int elt = w.kv_dtype == PTH_ATTN_F32 ? 4 : 2;
  const char* kr = w.key + tok * w.s_k_tok + static_cast<int64_t>(head) * w.s_k_head;
  const char* vr = w.value + tok * w.s_v_tok + static_cast<int64_t>(head) * w.s_v_head;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    xk[i] = load_elem(kr + static_cast<int64_t>(elt) * (NC * lane + i), w.kv_dtype);
    xv[i] = load_elem(vr + static_cast<int64_t>(elt) * (NC * lane + i), w.kv_dtype);
  }
  auto cell = [&](const CacheStream& s) {
    return const_cast<char*>(s.base) + page * s.s_block + in_page * s.s_slot +
           static_cast<int64_t>(head) * s.s_head;
  };
  quantize_row<NC>(xk, cell(w.k), reinterpret_cast<float*>(cell(w.ks)), lane);
  quantize_row<NC>(xv, cell(w.v), reinterpret_cast<float*>(cell(w.vs)), lane);
}

CacheStream stream_of(const PthAttnStream& s) {
  return CacheStream{static_cast<const char*>(s.data), s.stride_block, s.stride_slot,
                     s.stride_head};
}

}  // namespace

int32_t launch_write_kv(const PthAttnWriteArgs& a, hipStream_t stream) {
  clear_error();
  PA_REQUIRE(a.abi_version == PTH_ATTN_ABI_VERSION,
             "abi_version " + std::to_string(a.abi_version) + " != library ABI " +
                 std::to_string(PTH_ATTN_ABI_VERSION));
  PA_REQUIRE(a.struct_bytes == static_cast<int32_t>(sizeof(PthAttnWriteArgs)),
             "struct_bytes " + std::to_string(a.struct_bytes) + " != sizeof(PthAttnWriteArgs) " +
                 std::to_string(sizeof(PthAttnWriteArgs)));
  PA_REQUIRE(a.head_size == 64 || a.head_size == 128 || a.head_size == 256,
             "head_size must be 64, 128 or 256");
  PA_REQUIRE(a.kv_dtype == PTH_ATTN_F32 || a.kv_dtype == PTH_ATTN_F16 ||
                 a.kv_dtype == PTH_ATTN_BF16,
             "kv_dtype must be PTH_ATTN_F32, PTH_ATTN_F16 or PTH_ATTN_BF16");
  PA_REQUIRE(a.num_tokens >= 0 && a.num_kv_heads >= 1 && a.block_size >= 1 &&
                 a.num_blocks >= 1,
             "num_tokens >= 0, num_kv_heads, block_size and num_blocks >= 1");
  PA_REQUIRE(a.key && a.value && a.slot_mapping && a.k_cache.data && a.v_cache.data &&
                 a.k_scale.data && a.v_scale.data,
             "key, value, slot_mapping and the four cache streams must be non-NULL");
  const int64_t elt = a.kv_dtype == PTH_ATTN_F32 ? 4 : 2;
  PA_REQUIRE(reinterpret_cast<uintptr_t>(a.key) % elt == 0 &&
                 reinterpret_cast<uintptr_t>(a.value) % elt == 0 &&
                 a.key_stride_token % elt == 0 && a.key_stride_head % elt == 0 &&
                 a.value_stride_token % elt == 0 && a.value_stride_head % elt == 0,
             "key and value must be aligned to their element");
  PA_REQUIRE(reinterpret_cast<uintptr_t>(a.k_scale.data) % 4 == 0 &&
                 reinterpret_cast<uintptr_t>(a.v_scale.data) % 4 == 0 &&
                 a.k_scale.stride_slot % 4 == 0 && a.k_scale.stride_head % 4 == 0 &&
                 a.k_scale.stride_block % 4 == 0 && a.v_scale.stride_slot % 4 == 0 &&
                 a.v_scale.stride_head % 4 == 0 && a.v_scale.stride_block % 4 == 0,
             "the scale streams must be 4-B aligned");
  if (a.num_tokens == 0) return PTH_ATTN_OK;
  WriteParams w{};
  w.key = static_cast<const char*>(a.key);
  w.value = static_cast<const char*>(a.value);
  w.s_k_tok = a.key_stride_token;
  w.s_k_head = a.key_stride_head;
  w.s_v_tok = a.value_stride_token;
  w.s_v_head = a.value_stride_head;
  w.kv_dtype = a.kv_dtype;
  w.num_tokens = a.num_tokens;
  w.num_kv_heads = a.num_kv_heads;
  w.slot_mapping = a.slot_mapping;
  w.k = stream_of(a.k_cache);
  w.v = stream_of(a.v_cache);
  w.ks = stream_of(a.k_scale);
  w.vs = stream_of(a.v_scale);
  w.block_size = a.block_size;
  w.num_slots = static_cast<int64_t>(a.num_blocks) * a.block_size;
  const int64_t items = static_cast<int64_t>(a.num_tokens) * a.num_kv_heads;
  const dim3 grid(static_cast<unsigned>((items + 3) / 4)), block(256);
  switch (a.head_size) {
    case 64: hipLaunchKernelGGL(write_kv_int8<64>, grid, block, 0, stream, w); break;
    case 256: hipLaunchKernelGGL(write_kv_int8<256>, grid, block, 0, stream, w); break;
    default: hipLaunchKernelGGL(write_kv_int8<128>, grid, block, 0, stream, w);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(PTH_ATTN_ECUDA, std::string("cache writer launch: ") + hipGetErrorString(err));
  return PTH_ATTN_OK;
}

}  // namespace pa

extern "C" {

int32_t pth_attn_write_args_bytes(void) {
  return static_cast<int32_t>(sizeof(PthAttnWriteArgs));
}

int32_t pth_attn_write_kv(const PthAttnWriteArgs* args, void* stream) {
  if (args == nullptr) return pa::fail(PTH_ATTN_EINVAL, "args is NULL");
  return pa::launch_write_kv(*args, static_cast<hipStream_t>(stream));
}

}  // extern "C"
