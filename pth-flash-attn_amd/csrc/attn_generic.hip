// attn_generic.hip -- the gfx950 register-load attention kernel for any block
// size and any per-stream cache strides, head size D = 64, 128 or 256
// (reference instantiate_d*.cu: the op serves D in {64, 128, 256};
// sliding-window and non-causal attention at D = 128 only, reference
// launch.cu:301-310).
//
// The work decomposition, the MFMA layout and the numerics are those of the
// paged kernels (attn_fwd.hip, attn_device.h), with the per-lane layout
// scaled by D (HeadDim): lane (r, g) loads D/4 bytes of K per key, a V run
// of D/16 bytes per key, and holds D/4 output columns. Every key is looked up
// in the block table on its own, so pages of any size and caches whose four
// streams have unrelated strides (HND, padded pages, separate buffers) all
// work; the next chunk is loaded while the current one is computed.

#include "attn_device.h"

// Build switch: 0 sends every D = 256 launch to the register-load kernel
// (the comparison point of the direct-to-LDS D = 256 kernel below).
#ifndef PA_PAGED256
#define PA_PAGED256 1
#endif

namespace pa {
namespace {

// The cache bytes of one 32-key chunk for one lane, head size D.
template <int D>
struct ChunkD {
  uint32_t k[2][D / 16];  // K bytes [g D/4, (g + 1) D/4) of key 16 sub + r
  uint32_t v[8][D / 64];  // V bytes [r D/16, (r + 1) D/16) of key tv(e)
  float sc;               // one scale: k_scale (lanes r < 8) or v_scale of key tv(r % 8)
};

template <int D>
struct ChunkDOps {
  const ChunkD<D>& ch;
  __device__ __forceinline__ float sc() const { return ch.sc; }
  __device__ __forceinline__ bf16x8 k(int sub, int j) const {
    return i8x8_to_bf16(ch.k[sub][2 * j], ch.k[sub][2 * j + 1]);
  }
  // Byte j of each of the eight runs.
  __device__ __forceinline__ bf16x8 v(int j) const {
    const int w = j >> 2, b = j & 3;
    bf16x2 pr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      pr[e] = pack_bf16(i8_to_f32(ch.v[2 * e][w], b), i8_to_f32(ch.v[2 * e + 1][w], b));
    return (bf16x8){pr[0][0], pr[0][1], pr[1][0], pr[1][1], pr[2][0], pr[2][1], pr[3][0], pr[3][1]};
  }
};

// n bytes (a multiple of 4) at a 4-byte-aligned address into words.
template <int kWords>
__device__ __forceinline__ void load_words(const char* src, uint32_t* w) {
  if constexpr (kWords % 4 == 0) {
#pragma unroll
    for (int i = 0; i < kWords; i += 4) {
      const u32x4 x = *reinterpret_cast<const u32x4_a4*>(src + 4 * i);
      w[i] = x[0];
      w[i + 1] = x[1];
      w[i + 2] = x[2];
      w[i + 3] = x[3];
    }
  } else if constexpr (kWords == 2) {
    const u32x2 x = *reinterpret_cast<const u32x2_a4*>(src);
    w[0] = x[0];
    w[1] = x[1];
  } else {
    static_assert(kWords == 1, "1, 2 or a multiple of 4 words");
    w[0] = *reinterpret_cast<const uint32_t*>(src);
  }
}

// Chunk at key c of unit U; keys outside [ld_lo, ld_hi) are zero (they are
// masked in the softmax and never looked up in the block table).
template <int D>
__device__ __forceinline__ void load_chunk_d(const AttnParams& p, const Unit& U, const Lanes& L,
                                             int c, ChunkD<D>& ch) {
  const int BS = static_cast<int>(p.bs_div.d);
  const int32_t* bt = p.block_table + static_cast<int64_t>(U.t.req) * p.bt_stride;
  const int r16 = L.r16, g = L.g;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int tk = c + 16 * sub + r16;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) ch.k[sub][i] = 0u;
    if (tk >= U.ld_lo && tk < U.ld_hi) {
      const int blk = static_cast<int>(p.bs_div.div(tk));
      load_words<D / 16>(at(p.k, bt[blk], tk - blk * BS, U.kvh) + (D / 4) * g, ch.k[sub]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * sub + i;
      const int tv = c + 16 * sub + 4 * g + i;
#pragma unroll
      for (int w = 0; w < D / 64; ++w) ch.v[e][w] = 0u;
      if (tv >= U.ld_lo && tv < U.ld_hi) {
        const int blk = static_cast<int>(p.bs_div.div(tv));
        load_words<D / 64>(at(p.v, bt[blk], tv - blk * BS, U.kvh) + (D / 16) * r16, ch.v[e]);
      }
    }
  }
  const int e = r16 & 7;
  const int ts = c + 16 * (e >> 2) + 4 * g + (e & 3);
  float scv = 0.0f;
  if (ts >= U.ld_lo && ts < U.ld_hi) {
    const int blk = static_cast<int>(p.bs_div.div(ts));
    scv = *reinterpret_cast<const float*>(at(r16 < 8 ? p.ks : p.vs, bt[blk], ts - blk * BS, U.kvh));
  }
  ch.sc = scv;
}

template <bool kWindow, bool kStream, bool kF16Q, int D>
__global__ __launch_bounds__(kFwdWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_generic(const AttnParams p_arg) {
  // Two chunks in registers (one loading while the other is computed) while
  // they fit: 2 x 65 VGPRs at D = 256 do not, so D = 256 loads in turn.
  constexpr bool kDouble = D <= 128;
  const int lane = threadIdx.x & 63;
  const AttnParams p = params_in_registers(p_arg, lane);
  const float scl = scale_factor(lane & 15, p.scale_log2);
  Work<kWindow, kStream> work;
  work.init(p, lane);
  Unit U;
  while (work.next(p, lane, U)) {
    if (!U.has_rows) continue;
    const Lanes L = unit_lanes<kWindow>(p, U, lane);
    StateT<D> st;
    state_reset(st);
    if (U.n_chunks > 0) {
      bf16x8 qb[HeadDim<D>::kQK], qlo[HeadDim<D>::kQK];
      load_q<kF16Q, D>(p, L, qb, qlo);
      if constexpr (kDouble) {
        ChunkD<D> ca, cb;
        int k = 0;
        load_chunk_d<D>(p, U, L, U.c_begin, ca);
        while (true) {
          const int c = U.c_begin + kChunkTokens * k;
          if (k + 1 < U.n_chunks) load_chunk_d<D>(p, U, L, c + kChunkTokens, cb);
          compute_chunk_t<D, kF16Q>(U, L, c, ChunkDOps<D>{ca}, qb, qlo, scl, st);
          if (++k >= U.n_chunks) break;
          if (k + 1 < U.n_chunks) load_chunk_d<D>(p, U, L, c + 2 * kChunkTokens, ca);
          compute_chunk_t<D, kF16Q>(U, L, c + kChunkTokens, ChunkDOps<D>{cb}, qb, qlo, scl, st);
          if (++k >= U.n_chunks) break;
        }
      } else {
        for (int k = 0; k < U.n_chunks; ++k) {
          const int c = U.c_begin + kChunkTokens * k;
          ChunkD<D> ch;
          load_chunk_d<D>(p, U, L, c, ch);
          compute_chunk_t<D, kF16Q>(U, L, c, ChunkDOps<D>{ch}, qb, qlo, scl, st);
        }
      }
    }
    epilogue(p, U, L, st);
  }
}

// ---------------------------------------------------------------------------
// D = 256 on paged caches in the cell layout (block size a multiple of 16):
// the direct-to-LDS pipeline of attn_fwd_paged with 256-byte key rows. The
// chunk streams into one LDS slot per wave while the previous chunk, read
// out to registers, is computed; two chunks of D = 256 operands do not fit
// in registers, one plus an LDS slot does. A unit's chunk loop: wait for
// chunk k, read it out, issue chunk k + 1 into the slot, compute chunk k.
//
// Slot: K rows (32 x 256 B), V rows (32 x 256 B), then the 64 scales as in
// the D = 128 slot. The 16 pieces of 16 bytes of key row t are stored in the
// order piece ^ (t % 16): the K reads (16 keys, the same 4 pieces) and the V
// reads (one piece per lane of 16 keys) then touch distinct banks.
constexpr int kSlot256K = 0;
constexpr int kSlot256V = 32 * 256;
constexpr int kSlot256S = 64 * 256;
constexpr int kSlot256Bytes = 64 * 256 + 256;
constexpr int kDma256 = 17;  // 8 x 1 KB of K, 8 of V, the scales

__device__ __forceinline__ uint32_t swz256(int key, int piece) {
  return 256u * key + 16u * (piece ^ (key & 15));
}

// Per-lane byte offsets within a 16-key group of one page (the cell view):
// DMA q (0 .. 3) of a group covers keys 4q .. 4q + 3; lane l loads piece
// (l % 16) ^ key of key 4q + l / 16, so it lands in its swizzled position.
struct Prod256 {
  uint32_t off_k[4];
  uint32_t dv;     // V offset minus K offset (uniform)
  uint32_t off_s;
  int32_t page[2], slot0[2];
};

__device__ __forceinline__ void prod256_offsets(const AttnParams& p, const Unit& U, int lane,
                                                Prod256& P) {
  const uint32_t head = static_cast<uint32_t>(U.kvh) * p.cell_head;
  const uint32_t pos = lane & 15, kr = lane >> 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t key = 4u * q + kr;
    P.off_k[q] = key * p.cell_slot + head + p.cell_off[0] + 16u * (pos ^ key);
  }
  P.dv = p.cell_off[1] - p.cell_off[0];
  P.off_s = static_cast<uint32_t>(lane & 15) * p.cell_slot + head +
            (lane < 32 ? p.cell_off[2] : p.cell_off[3]);
}

__device__ __forceinline__ void prod256_pages(const AttnParams& p, const Unit& U, int c,
                                              Prod256& P) {
  // The unit is wave-uniform; saying so makes the block-table reads scalar
  // loads (lgkmcnt), which never wait for the chunk loads in flight.
  const int req = __builtin_amdgcn_readfirstlane(U.t.req);
  const int ld_lo = __builtin_amdgcn_readfirstlane(U.ld_lo);
  const int ld_hi = __builtin_amdgcn_readfirstlane(U.ld_hi);
  c = __builtin_amdgcn_readfirstlane(c);
  const int64_t bt0 = static_cast<int64_t>(req) * p.bt_stride;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int c16 = c + 16 * sub;
    P.page[sub] = 0;
    P.slot0[sub] = 0;
    if (c16 < ld_hi && c16 + 16 > ld_lo) {
      const int blk = static_cast<int>(p.bs_div.div(c16));
      P.slot0[sub] = c16 - blk * static_cast<int>(p.bs_div.d);
      P.page[sub] = ld_ro(p.block_table, bt0 + blk);
    }
  }
}

// The 17 direct-to-LDS loads of the chunk whose pages P holds. Every address
// is inside the cache (keys outside the unit's range are masked later).
__device__ __forceinline__ void issue256(const AttnParams& p, const Prod256& P, char* slot,
                                         int lane) {
  const char* base[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    base[sub] = p.cell_base +
                static_cast<uint64_t>(static_cast<uint32_t>(P.page[sub])) * p.cell_block +
                static_cast<uint32_t>(P.slot0[sub]) * p.cell_slot;
#pragma unroll
  for (int i = 0; i < 8; ++i) dma16(base[i >> 2] + P.off_k[i & 3], slot + kSlot256K + 1024 * i);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    dma16(base[i >> 2] + P.off_k[i & 3] + P.dv, slot + kSlot256V + 1024 * i);
  dma4(((lane >> 4) & 1 ? base[1] : base[0]) + P.off_s, slot + kSlot256S);
}

// Chunk in LDS -> the lane's operands (the layout of ChunkD<256>): K bytes
// [64 g, 64 g + 64) of keys r and 16 + r, V bytes [16 r, 16 r + 16) of keys
// tv(e), one scale. Returns once the reads have landed.
__device__ __forceinline__ void read256(uint32_t slot, int lane, ChunkD<256>& ch) {
  const int r16 = lane & 15, g = lane >> 4;
  u32x4 kk[2][4], vv[8];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = slot + kSlot256K + swz256(16 * sub + r16, 4 * g + i);
      asm volatile("ds_read_b128 %0, %1" : "=v"(kk[sub][i]) : "v"(a));
    }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int tv = 16 * (e >> 2) + 4 * g + (e & 3);
    const uint32_t a = slot + kSlot256V + swz256(tv, r16);
    asm volatile("ds_read_b128 %0, %1" : "=v"(vv[e]) : "v"(a));
  }
  const int e = r16 & 7;
  const int key = 16 * (e >> 2) + 4 * g + (e & 3);
  float sc;
  asm volatile("ds_read_b32 %0, %1"
               : "=v"(sc)
               : "v"(slot + kSlot256S + (r16 < 8 ? 0u : 128u) + 4u * key));
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(kk[0][0]), "+v"(kk[0][1]), "+v"(kk[0][2]), "+v"(kk[0][3]),
                 "+v"(kk[1][0]), "+v"(kk[1][1]), "+v"(kk[1][2]), "+v"(kk[1][3]), "+v"(vv[0]),
                 "+v"(vv[1]), "+v"(vv[2]), "+v"(vv[3]), "+v"(vv[4]), "+v"(vv[5]), "+v"(vv[6]),
                 "+v"(vv[7]), "+v"(sc)
               :
               : "memory");
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t x = kk[sub][i][w];
        ch.k[sub][4 * i + w] = x;
      }
#pragma unroll
  for (int e2 = 0; e2 < 8; ++e2)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t x = vv[e2][w];
      ch.v[e2][w] = x;
    }
  ch.sc = sc;
}

template <bool kStream, bool kF16Q>
__global__ __launch_bounds__(kFwdWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_paged256(const AttnParams p_arg) {
  constexpr int D = 256;
  __shared__ __attribute__((aligned(16))) char lds_all[kFwdWaves * kSlot256Bytes];
  const int lane = threadIdx.x & 63;
  const AttnParams p = params_in_registers(p_arg, lane);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char* slot = lds_all + wave * kSlot256Bytes;
  const uint32_t slot_a = lds_offset(slot);
  const float scl = scale_factor(lane & 15, p.scale_log2);
  Work<false, kStream> work;
  work.init(p, lane);
  Unit U;
  while (work.next(p, lane, U)) {
    if (!U.has_rows) continue;
    const Lanes L = unit_lanes<false>(p, U, lane);
    StateT<D> st;
    state_reset(st);
    if (U.n_chunks > 0) {
      Prod256 P;
      prod256_offsets(p, U, lane, P);
      prod256_pages(p, U, U.c_begin, P);
      issue256(p, P, slot, lane);
      if (U.n_chunks > 1) prod256_pages(p, U, U.c_begin + kChunkTokens, P);
      bf16x8 qb[HeadDim<D>::kQK], qlo[HeadDim<D>::kQK];
      load_q<kF16Q, D>(p, L, qb, qlo);
      // The query and chunk 0 (compiler-visible vmcnt(0)).
      __builtin_amdgcn_s_waitcnt(0x0F70);
      for (int k = 0; k < U.n_chunks; ++k) {
        const int c = U.c_begin + kChunkTokens * k;
        wait_vmcnt<0>();  // chunk k has landed (the only loads in flight)
        ChunkD<D> ch;
        read256(slot_a, lane, ch);
        if (k + 1 < U.n_chunks) {
          issue256(p, P, slot, lane);
          if (k + 2 < U.n_chunks) prod256_pages(p, U, c + 2 * kChunkTokens, P);
        }
        compute_chunk_t<D, kF16Q>(U, L, c, ChunkDOps<D>{ch}, qb, qlo, scl, st);
      }
    }
    epilogue(p, U, L, st);
  }
}

bool use_paged256(const AttnParams& p) { return p.cell && p.bs_div.d % 16 == 0; }

template <bool W, bool St, int D>
hipError_t launch_d(const AttnParams& p, dim3 grid, bool q_f16, hipStream_t stream) {
  if (q_f16)
    hipLaunchKernelGGL((attn_fwd_generic<W, St, true, D>), grid, dim3(kFwdWaves * 64), 0, stream,
                       p);
  else
    hipLaunchKernelGGL((attn_fwd_generic<W, St, false, D>), grid, dim3(kFwdWaves * 64), 0, stream,
                       p);
  return hipGetLastError();
}

template <bool St>
hipError_t launch_paged256(const AttnParams& p, dim3 grid, bool q_f16, hipStream_t stream) {
  if (q_f16)
    hipLaunchKernelGGL((attn_fwd_paged256<St, true>), grid, dim3(kFwdWaves * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((attn_fwd_paged256<St, false>), grid, dim3(kFwdWaves * 64), 0, stream, p);
  return hipGetLastError();
}

template <int D>
hipError_t launch_causal(const AttnParams& p, dim3 grid, bool q_f16, hipStream_t stream) {
  if (D == 256 && PA_PAGED256 && use_paged256(p))
    return p.num_splits > 1 ? launch_paged256<true>(p, grid, q_f16, stream)
                            : launch_paged256<false>(p, grid, q_f16, stream);
  return p.num_splits > 1 ? launch_d<false, true, D>(p, grid, q_f16, stream)
                          : launch_d<false, false, D>(p, grid, q_f16, stream);
}

}  // namespace

hipError_t launch_generic_kernel(const AttnParams& p, dim3 grid, bool windowed, bool q_f16,
                                 int head_size, hipStream_t stream) {
  const bool split = p.num_splits > 1;
  switch (head_size) {
    case 64:
      if (windowed) return hipErrorInvalidValue;
      return launch_causal<64>(p, grid, q_f16, stream);
    case 256:
      if (windowed) return hipErrorInvalidValue;
      return launch_causal<256>(p, grid, q_f16, stream);
    default:
      if (windowed)
        return split ? launch_d<true, true, 128>(p, grid, q_f16, stream)
                     : launch_d<true, false, 128>(p, grid, q_f16, stream);
      return launch_causal<128>(p, grid, q_f16, stream);
  }
}

}  // namespace pa
