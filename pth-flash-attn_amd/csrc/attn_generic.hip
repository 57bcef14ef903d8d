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
void attn_fwd_generic(const AttnParams p) {
  // Two chunks in registers (one loading while the other is computed) while
  // they fit: 2 x 65 VGPRs at D = 256 do not, so D = 256 loads in turn.
  constexpr bool kDouble = D <= 128;
  const int lane = threadIdx.x & 63;
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

template <int D>
hipError_t launch_causal(const AttnParams& p, dim3 grid, bool q_f16, hipStream_t stream) {
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
