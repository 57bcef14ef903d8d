// read_ceiling.hip -- achievable HBM read bandwidth on one MI355X for the paged
// cell layout of the attention kernels (8 KV heads x 264-byte cells, pages of
// 16 tokens, a shuffled page order over ~2.2 GB). Each variant reads every
// byte of every page once and discards it:
//   * head: per-head cells as the attention kernels read them (register
//     loads of K, V and the scales of one head per wave, U 16-token groups
//     in flight);
//   * rows: whole pages (33 contiguous KB) per wave, P loads in flight;
//   * rows pipe: whole pages, the next page's 33 loads issued before the
//     current one is consumed;
//   * dma: per-head cells by direct-to-LDS loads as the paged kernel issues
//     them (C 16-key groups per chunk, D chunks in flight per wave, and a
//     work-group barrier every BAR chunks when BAR > 0).
// Not part of the library: a measurement of the ceiling that the kernels'
// roofline fractions are read against.
//
// Build and run (from the repository root, on the GPU):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     pth-flash-attn_amd/probes/read_ceiling.hip -o /tmp/read_ceiling && /tmp/read_ceiling
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#include <random>
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
#define CK(x) do{hipError_t e=(x); if(e!=hipSuccess){printf("err %s line %d\n",hipGetErrorString(e),__LINE__);exit(1);}}while(0)
constexpr int PAGE = 16 * 8 * 264;  // 33792 = 33 KB

__device__ __forceinline__ void dma16(const char* g, char* lds) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(g),
      (void __attribute__((address_space(3)))*)(lds), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const char* g, char* lds) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(g),
      (void __attribute__((address_space(3)))*)(lds), 4, 0, 0);
}
template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }

// DMA: per wave (= head) a sequence of 16-key groups (one page each). A "chunk" = C groups
// (C = 1: 16 keys, 5 DMAs; C = 2: 32 keys, 9 DMAs). D chunks in flight.
template <int C, int D, bool SWZ = false, int BAR = 0>
__global__ __launch_bounds__(512) void rd_dma(const char* base, const int* pages, int npages, int per_wg, uint32_t* out) {
  constexpr int SLOT = C * 16 * 264;
  __shared__ __attribute__((aligned(16))) char lds_all[8 * D * SLOT];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  char* lds = lds_all + wave * D * SLOT;
  const int pb = blockIdx.x * per_wg, pe = min(npages, pb + per_wg);
  const int tok = lane >> 3, piece = lane & 7;
  uint32_t acc = 0;
  auto issue = [&](int pg, char* slot) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int pgi = min(pg + c, pe - 1);
      const char* page = base + (size_t)pages[pgi] * PAGE;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const char* cell = page + (size_t)(8 * h + tok) * 2112 + wave * 264;
        const int pc = SWZ ? (piece ^ tok) : piece;
        dma16(cell + 16 * pc, slot + c * 4096 + 1024 * h);
        dma16(cell + 132 + 16 * pc, slot + c * 4096 + 2048 + 1024 * h);
      }
    }
    // scales: lanes 0..15: ks of keys 0..15 of group 0, 16..31 vs; 32.. group 1 (C=2)
    const int c = C == 2 ? (lane >> 5) : 0;
    const int pgi = min(pg + c, pe - 1);
    const char* page = base + (size_t)pages[pgi] * PAGE;
    if (C == 2 || lane < 32)
      dma4(page + (size_t)(lane & 15) * 2112 + wave * 264 + ((lane & 16) ? 260 : 128), slot + C * 4096);
  };
  int pg = pb, inflight = 0, slot_w = 0, slot_r = 0;
  for (int i = 0; i < D && pg < pe; ++i) { issue(pg, lds + slot_w * SLOT); pg += C; ++inflight; slot_w = (slot_w + 1) % D; }
  while (inflight > 0) {
    if (inflight >= 2 && D >= 2) wait_vm<(C == 2 ? 9 : 5)>(); else wait_vm<0>();
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : "=v"(v) : "v"((uint32_t)(uintptr_t)(lds + slot_r * SLOT + 4 * lane)));
    acc ^= v;
    --inflight; slot_r = (slot_r + 1) % D;
    if (pg < pe) { issue(pg, lds + slot_w * SLOT); pg += C; ++inflight; slot_w = (slot_w + 1) % D; }
    if (BAR > 0 && ((pg - pb) / C) % BAR == 0) __builtin_amdgcn_s_barrier();
  }
  if (acc == 0x12345678) out[0] = acc;
}

// per-head cell reads (the current kernel's pattern), register loads, U groups in flight
template <int U>
__global__ __launch_bounds__(512) void rd_head(const char* base, const int* pages, int npages, int per_wg, uint32_t* out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pb = blockIdx.x * per_wg, pe = min(npages, pb + per_wg);
  uint32_t acc = 0;
  const int tok = lane >> 3, piece = lane & 7;
  for (int pg = pb; pg < pe; pg += U) {
    u32x4 k[U][2], v[U][2];
    uint32_t s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pgi = min(pg + u, pe - 1);
      const char* page = base + (size_t)pages[pgi] * PAGE;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const char* cell = page + (size_t)(8 * h + tok) * 2112 + wave * 264;
        k[u][h] = *(const u32x4a*)(cell + 16 * piece);
        v[u][h] = *(const u32x4a*)(cell + 132 + 16 * piece);
      }
      s[u] = *(const uint32_t*)(page + (size_t)(lane & 15) * 2112 + wave * 264 + (lane < 16 ? 128 : 260));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= k[u][0].x ^ k[u][1].y ^ v[u][0].z ^ v[u][1].w ^ s[u];
  }
  if (acc == 0x12345678) out[0] = acc;
}

// whole-page (token-row) reads: wave w of the work-group reads pages pb + w, + 8, ...;
// a page is 33 contiguous KB: 33 loads of 16 B per lane. P loads per batch in flight.
template <int P>
__global__ __launch_bounds__(512) void rd_rows(const char* base, const int* pages, int npages, int per_wg, uint32_t* out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pb = blockIdx.x * per_wg, pe = min(npages, pb + per_wg);
  uint32_t acc = 0;
  for (int pg = pb + wave; pg < pe; pg += 8) {
    const char* page = base + (size_t)pages[pg] * PAGE + 16 * lane;
    for (int i0 = 0; i0 < 33; i0 += P) {
      u32x4 x[P];
#pragma unroll
      for (int i = 0; i < P; ++i) x[i] = i0 + i < 33 ? *(const u32x4a*)(page + 1024 * (i0 + i)) : (u32x4){0,0,0,0};
#pragma unroll
      for (int i = 0; i < P; ++i) acc ^= x[i].x ^ x[i].w;
    }
  }
  if (acc == 0x12345678) out[0] = acc;
}

// whole pages, all 33 loads of a page in flight, next page's loads issued before consuming
__global__ __launch_bounds__(512) void rd_rows_pipe(const char* base, const int* pages, int npages, int per_wg, uint32_t* out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pb = blockIdx.x * per_wg, pe = min(npages, pb + per_wg);
  uint32_t acc = 0;
  u32x4 a[33];
  int pg = pb + wave;
  if (pg < pe) {
    const char* page = base + (size_t)pages[pg] * PAGE + 16 * lane;
#pragma unroll
    for (int i = 0; i < 33; ++i) a[i] = *(const u32x4a*)(page + 1024 * i);
  }
  for (; pg < pe; pg += 8) {
#pragma unroll
    for (int i = 0; i < 33; ++i) acc ^= a[i].x ^ a[i].w;
    const int nx = pg + 8;
    if (nx < pe) {
      const char* page = base + (size_t)pages[nx] * PAGE + 16 * lane;
#pragma unroll
      for (int i = 0; i < 33; ++i) a[i] = *(const u32x4a*)(page + 1024 * i);
    }
  }
  if (acc == 0x12345678) out[0] = acc;
}

int main() {
  const int npages = 66000;  // ~2.23 GB
  size_t bytes = (size_t)npages * PAGE;
  char* buf; uint32_t* out; int* pages;
  CK(hipMalloc(&buf, bytes)); CK(hipMalloc(&out, 64)); CK(hipMalloc(&pages, npages * 4));
  CK(hipMemset(buf, 1, bytes));
  std::vector<int> perm(npages); for (int i = 0; i < npages; ++i) perm[i] = i;
  std::mt19937 rng(1); std::shuffle(perm.begin(), perm.end(), rng);
  CK(hipMemcpy(pages, perm.data(), npages * 4, hipMemcpyHostToDevice));
  hipEvent_t a, b; CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
  int cus = 0; CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  auto timeit = [&](const char* name, auto launch) {
    launch(); CK(hipDeviceSynchronize());
    CK(hipEventRecord(a));
    for (int i = 0; i < 10; ++i) launch();
    CK(hipEventRecord(b)); CK(hipEventSynchronize(b));
    float ms; CK(hipEventElapsedTime(&ms, a, b));
    printf("%-40s %8.1f us  %7.0f GB/s\n", name, ms * 100, bytes / (ms * 1e-4) / 1e9);
  };
  int grid = cus; int per = (npages + grid - 1) / grid;
  timeit("head reg U=1", [&]{ rd_head<1><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("head reg U=2", [&]{ rd_head<2><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("rows P=4", [&]{ rd_rows<4><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("rows P=11", [&]{ rd_rows<11><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("rows P=33", [&]{ rd_rows<33><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("rows pipe 2x33", [&]{ rd_rows_pipe<<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("dma C=2 D=1", [&]{ rd_dma<2,1><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("dma C=2 D=2", [&]{ rd_dma<2,2><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("dma C=2 D=2 swizzled", [&]{ rd_dma<2,2,true><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("dma C=2 D=1, barrier every 8 chunks", [&]{ rd_dma<2,1,false,8><<<grid,512>>>(buf, pages, npages, per, out); });
  timeit("dma C=2 D=1, 2 work-groups per CU", [&]{ rd_dma<2,1><<<2*grid,512>>>(buf, pages, npages, (npages + 2*grid - 1)/(2*grid), out); });
  timeit("dma C=2 D=1, 3 work-groups per CU", [&]{ rd_dma<2,1><<<3*grid,512>>>(buf, pages, npages, (npages + 3*grid - 1)/(3*grid), out); });
  timeit("rows P=11 grid x2", [&]{ rd_rows<11><<<2*grid,512>>>(buf, pages, npages, (npages + 2*grid - 1)/(2*grid), out); });
  return 0;
}
