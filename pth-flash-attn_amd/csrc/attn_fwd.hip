// attn_fwd.hip -- the gfx950 paged int8 attention kernels, D = 128: the work
// decomposition and MFMA layout they share, the register-load kernel for
// short windows, and the dispatch between it and the register-staged
// kernels of attn_staged.hip (long rows).
//
// Work decomposition. A work unit is (request, row tile, KV head, 16-row
// group) over a range of keys; a row tile holds up to bq query tokens of one
// request and its rows are (token, head-in-group) pairs, token-major
// (reference cache_geometry.cuh:319-334). The kernels are persistent and
// derive their work on the device from query_start_loc and seq_lens, so a
// launch is graph-safe (Work in attn_device.h). With one split, wave w of
// the grid takes units w, w + W, ... of a table built by a prefix sum over
// the requests. With S > 1, the 32-key chunk streams of every (row tile,
// group of 8 KV-head units) are laid end to end and work-group b takes the
// positions [b per, (b + 1) per) (attn_geometry.h, attn_stream.h), so every
// work-group has the same work and a stream has as many splits as the
// work-groups it meets (at most the planner's S). The 8 waves of a
// work-group take the 8 units of a group: with 8 KV heads, the 8 heads of
// the same keys, whose cells are adjacent in memory and share cache lines.
//
// MFMA layout ("swap AB"). Both products use v_mfma_f32_16x16x32_bf16 with the
// keys on the M side and the 16 query rows on N:
//   S^T[key][row]  = K[key][d]   * Q^T[d][row]     (4 MFMAs per 16 keys)
//   O^T[d][row]   += V^T[d][key] * P^T[key][row]   (8 MFMAs per 32 keys)
// so lane l always holds query row (l % 16): its softmax state, its scores,
// its probabilities and 32 contiguous output columns d in [32 g, 32 g + 32),
// g = l / 16. No cross-lane transpose is needed anywhere: the MFMA's K index
// may be permuted freely as long as A and B agree, and the choices below
// make every lane read whole byte runs of the cache:
//   * K: lane (r, g) reads bytes [32 g, 32 g + 32) of key r of a 16-key block;
//   * V: lane (m, g) reads bytes [8 m, 8 m + 8) of the 8 keys
//     {4 g + i, 16 + 4 g + i : i < 4} of a 32-key chunk, and MFMA j takes byte
//     j of each, so the 8 x 8 byte transpose happens for free in the byte
//     select of the int8 -> fp32 conversion;
//   * the keys of the score tile that lane (r, g) holds after QK are exactly
//     those keys, in the same order, so P feeds PV straight from registers.
//
// Dequantisation. int8 -> fp32 is v_cvt_f32_i32 with a sign-extending byte
// select, then v_cvt_pk_bf16_f32 packs two; both exact (|x| <= 128 needs 8
// significant bits). K's scale multiplies the fp32 score after QK and V's
// scale is folded into P before it is rounded to bf16 (reference
// attn_kernel.cuh:566-575, softmax.cuh:163-168). bf16 shares fp32's exponent
// range, so neither the reference's Q prescale nor its V-scale exponent is
// needed (they exist for fp16's range).
//
// Softmax. Scores are in log2 units (scale * log2 e folded in); the running
// max is reduced over the 4 lanes of a row with the gfx950 cross-row swaps
// (permlane16/32); the running sum stays per lane and is reduced once at the
// end.

#include "attn_device.h"

namespace pa {
namespace {

// ---------------------------------------------------------------------------
// Paged kernel with register loads (block size a multiple of 16, cell view of
// the cache): each lane loads exactly the bytes of its MFMA operands (the
// layout read_chunk produces from LDS) straight into registers, the next
// chunk's loads in flight while the current chunk is computed; page numbers
// are looked up one chunk ahead on the scalar unit.
struct RegLoader {
  int32_t page[2], slot0[2];  // pages of the chunk to load next
  uint32_t off_k, off_v[4], off_s;
};

__device__ __forceinline__ void reg_offsets(const AttnParams& p, const Unit& U, int lane,
                                            RegLoader& R) {
  const uint32_t r16 = lane & 15, g = lane >> 4;
  const uint32_t head = static_cast<uint32_t>(U.kvh) * p.cell_head;
  R.off_k = r16 * p.cell_slot + head + 32u * g + p.cell_off[0];
#pragma unroll
  for (int q = 0; q < 4; ++q) R.off_v[q] = (4u * g + q) * p.cell_slot + head + p.cell_off[1] + 8u * r16;
  const uint32_t e = r16 & 7;
  R.off_s = (4u * g + (e & 3)) * p.cell_slot + head + (r16 < 8 ? p.cell_off[2] : p.cell_off[3]);
}

__device__ __forceinline__ void reg_pages(const AttnParams& p, const Unit& U, int c,
                                          RegLoader& R) {
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
    R.page[sub] = 0;
    R.slot0[sub] = 0;
    if (c16 < ld_hi && c16 + 16 > ld_lo) {
      const int blk = static_cast<int>(p.bs_div.div(c16));
      R.slot0[sub] = c16 - blk * static_cast<int>(p.bs_div.d);
      R.page[sub] = ld_ro(p.block_table, bt0 + blk);
    }
  }
}

__device__ __forceinline__ void reg_load(const AttnParams& p, const RegLoader& R, int lane,
                                         Chunk& ch) {
  const char* base[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    base[sub] = p.cell_base +
                static_cast<uint64_t>(static_cast<uint32_t>(R.page[sub])) * p.cell_block +
                static_cast<uint32_t>(R.slot0[sub]) * p.cell_slot;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    ch.k[sub][0] = *reinterpret_cast<const u32x4_a4*>(base[sub] + R.off_k);
    ch.k[sub][1] = *reinterpret_cast<const u32x4_a4*>(base[sub] + R.off_k + 16);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) ch.v[e] = *reinterpret_cast<const u32x2_a4*>(base[e >> 2] + R.off_v[e & 3]);
  const char* sb = ((lane & 7) >> 2) ? base[1] : base[0];
  ch.sc = *reinterpret_cast<const float*>(sb + R.off_s);
}

template <bool kWindow, bool kStream, bool kF16Q>
__global__ __launch_bounds__(kFwdWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_paged_reg(const AttnParams p_arg) {
  const int lane = threadIdx.x & 63;
  const AttnParams p = params_in_registers(p_arg, lane);
  const float scl = scale_factor(lane & 15, p.scale_log2);
  Work<kWindow, kStream> work;
  work.init(p, lane);
  Unit U;
  while (work.next(p, lane, U)) {
    if (!U.has_rows) continue;
    const Lanes L = unit_lanes<kWindow>(p, U, lane);
    State st;
    state_reset(st);
    if (U.n_chunks > 0) {
      RegLoader R;
      reg_offsets(p, U, lane, R);
      reg_pages(p, U, U.c_begin, R);
      Chunk ca, cb;
      reg_load(p, R, lane, ca);
      if (U.n_chunks > 1) reg_pages(p, U, U.c_begin + kChunkTokens, R);
      bf16x8 qb[4], qlo[4];
      load_q<kF16Q>(p, L, qb, qlo);
      int k = 0;
      while (true) {
        const int c = U.c_begin + kChunkTokens * k;
        if (k + 1 < U.n_chunks) {
          reg_load(p, R, lane, cb);
          if (k + 2 < U.n_chunks) reg_pages(p, U, c + 2 * kChunkTokens, R);
        }
        compute_chunk<kF16Q>(U, L, c, ca, qb, qlo, scl, st);
        if (++k >= U.n_chunks) break;
        if (k + 1 < U.n_chunks) {
          reg_load(p, R, lane, ca);
          if (k + 2 < U.n_chunks) reg_pages(p, U, c + 3 * kChunkTokens, R);
        }
        compute_chunk<kF16Q>(U, L, c + kChunkTokens, cb, qb, qlo, scl, st);
        if (++k >= U.n_chunks) break;
      }
    }
    epilogue(p, U, L, st);
  }
}

// Windows up to this many keys: the register-load kernel (its short
// latency wins when every row reads few keys); otherwise the register-staged
// kernels of attn_staged.hip (the higher sustained bandwidth on long rows).
constexpr int kShortWindow = 4096;

template <bool W, bool St, bool F>
hipError_t launch_paged(const AttnParams& p, dim3 grid, hipStream_t stream) {
  if (W && p.window > 0 && p.window <= kShortWindow) {
    hipLaunchKernelGGL((attn_fwd_paged_reg<W, St, F>), grid, dim3(kFwdWaves * 64), 0, stream, p);
    return hipGetLastError();
  }
  return launch_staged_kernel(p, grid, W, F, stream);
}
template <bool W, bool St>
hipError_t launch_variant(const AttnParams& p, dim3 grid, bool q_f16, hipStream_t stream) {
  return q_f16 ? launch_paged<W, St, true>(p, grid, stream)
               : launch_paged<W, St, false>(p, grid, stream);
}

}  // namespace

hipError_t launch_fwd_kernel(const AttnParams& p, dim3 grid, bool windowed,
                             bool paged16, bool q_f16, hipStream_t stream) {
  if (!paged16) return launch_generic_kernel(p, grid, windowed, q_f16, 128, stream);
  const bool stream_split = p.num_splits > 1;
  if (windowed) return stream_split ? launch_variant<true, true>(p, grid, q_f16, stream)
                                    : launch_variant<true, false>(p, grid, q_f16, stream);
  return stream_split ? launch_variant<false, true>(p, grid, q_f16, stream)
                      : launch_variant<false, false>(p, grid, q_f16, stream);
}

}  // namespace pa
