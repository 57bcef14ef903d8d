// ceilings.hip -- the measured ceilings bench.py reports beside MI355X's
// nominal peaks (libpth_bench.so, built by __graft_entry__.build(); not part
// of the attention library). The reference measures the same two things
// (bench/sol_copy.cu: read the kernel's bytes and discard them;
// bench/mma_ceiling.cu: the tensor-core ceiling at the kernel's occupancy).
//
//  * pth_bench_read_groups: reads exactly the cache bytes of a decode
//    launch -- for each (page, slots) entry the first `slots` slot rows of
//    one 16-slot group of a page -- with the attention kernel's load
//    pattern (work-groups of 512 lanes, whole slot rows in 16-byte register
//    loads with the non-temporal hint, two groups in flight per work-group,
//    static equal ranges of entries per work-group) and discards them. Its GB/s is the achievable
//    read rate of that byte set.
//  * pth_bench_mfma: back-to-back v_mfma_f32_16x16x32_bf16 on 8 waves per CU
//    (2 per SIMD, the row-block kernel's occupancy), 8 independent
//    accumulators per wave. Its TFLOP/s is the dense bf16 MFMA ceiling.
//
// Both return the average milliseconds of `reps` launches (HIP events on
// `stream`) or a negative HIP error code.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One group entry: page index and the number of its slots the launch reads.
struct Group {
  int32_t page;
  int32_t slots;
};

__global__ __launch_bounds__(512) void read_groups(const char* base, int64_t page_bytes,
                                                   int32_t slot0_bytes, int32_t row_bytes,
                                                   const Group* groups, int32_t n_groups,
                                                   int32_t per_wg, uint32_t* sink) {
  const int L = threadIdx.x;
  const int g0 = blockIdx.x * per_wg;
  const int g1 = min(n_groups, g0 + per_wg);
  const int pieces_per_row = row_bytes / 16;
  uint32_t acc = 0;
  for (int g = g0; g < g1; g += 2) {
    u32x4 v[2][5];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int gi = g + h < g1 ? g + h : g;
      const Group e = groups[gi];
      const int n = g + h < g1 ? e.slots * pieces_per_row : 0;
      const char* src = base + static_cast<int64_t>(e.page) * page_bytes + slot0_bytes;
#pragma unroll
      for (int j = 0; j < 5; ++j) {
        const int i = L + 512 * j;
        v[h][j] = i < n ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16 * i))
                        : (u32x4){0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 5; ++j) acc ^= v[h][j].x ^ v[h][j].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads; practically never true
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfma_loop(int32_t iters, float* sink) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = static_cast<__bf16>(0.001f * (lane + e));
    b[e] = static_cast<__bf16>(0.002f * (lane - e));
  }
  f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[k], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
  if (s == 12345.678f) sink[0] = s;
}

template <class Launch>
float time_launches(int reps, hipStream_t stream, Launch launch, hipError_t* err) {
  hipEvent_t e0, e1;
  *err = hipEventCreate(&e0);
  if (*err != hipSuccess) return -1.f;
  *err = hipEventCreate(&e1);
  if (*err != hipSuccess) {
    hipEventDestroy(e0);
    return -1.f;
  }
  float ms = 0.f;
  launch();  // untimed
  *err = hipGetLastError();
  if (*err == hipSuccess) *err = hipEventRecord(e0, stream);
  if (*err == hipSuccess) {
    for (int i = 0; i < reps; ++i) launch();
    *err = hipGetLastError();
  }
  if (*err == hipSuccess) *err = hipEventRecord(e1, stream);
  if (*err == hipSuccess) *err = hipEventSynchronize(e1);
  if (*err == hipSuccess) *err = hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  return *err == hipSuccess ? ms / reps : -1.f;
}

}  // namespace

extern "C" {

// groups: device array of n_groups (page, slots) int32 pairs; slots <= 16
// and slot0_bytes + 16 slot rows lie inside each page. sink: 4 device bytes.
float pth_bench_read_groups(const void* base, int64_t page_bytes, int32_t slot0_bytes,
                            int32_t row_bytes, const void* groups, int32_t n_groups,
                            int32_t num_wg, void* sink, int32_t reps, void* stream) {
  if (base == nullptr || groups == nullptr || sink == nullptr || n_groups < 1 || num_wg < 1 ||
      reps < 1 || row_bytes % 16 != 0 || 16 * row_bytes > 5 * 512 * 16)
    return -1.f;
  const int32_t per = ((n_groups + num_wg - 1) / num_wg + 1) & ~1;  // even: groups go in pairs
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t err;
  const float ms = time_launches(reps, st, [&] {
    hipLaunchKernelGGL(read_groups, dim3(num_wg), dim3(512), 0, st,
                       static_cast<const char*>(base), page_bytes, slot0_bytes, row_bytes,
                       static_cast<const Group*>(groups), n_groups, per,
                       static_cast<uint32_t*>(sink));
  }, &err);
  return err == hipSuccess ? ms : -static_cast<float>(err);
}

// Flops of one launch: num_wg * 8 waves * iters * 8 MFMAs * 16 * 16 * 32 * 2.
float pth_bench_mfma(int32_t num_wg, int32_t iters, void* sink, int32_t reps, void* stream) {
  if (num_wg < 1 || iters < 1 || sink == nullptr || reps < 1) return -1.f;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t err;
  const float ms = time_launches(reps, st, [&] {
    hipLaunchKernelGGL(mfma_loop, dim3(num_wg), dim3(512), 0, st, iters,
                       static_cast<float*>(sink));
  }, &err);
  return err == hipSuccess ? ms : -static_cast<float>(err);
}

}  // extern "C"
