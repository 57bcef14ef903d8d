// attn_fwd.hip -- the gfx950 paged int8 attention kernel, D = 128.
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

#ifndef PA_REG_REALIGN
#define PA_REG_REALIGN 0
#endif
#ifndef PA_DECODE_REG
#define PA_DECODE_REG 0
#endif
#ifndef PA_PAGED_INFLIGHT
#define PA_PAGED_INFLIGHT 1
#endif

namespace pa {
namespace {

// ---------------------------------------------------------------------------
// Paged kernel (block size a multiple of 16): the 16-key halves of a chunk
// each lie in one page. A producer walks this wave's chunk sequence -- all
// chunks of its units, in order -- and keeps the next PA_PAGED_INFLIGHT chunks
// in flight in the wave's LDS slots with direct-to-LDS loads; the consumer
// computes the chunk before them from registers. One slot is the default: the
// consumer copies a chunk to registers, refills the slot and computes while
// the next chunk loads. A second slot (two chunks in flight) measured 1-3 %
// slower on the long-decode configurations: the deeper queue of DMA writes
// into LDS costs more than the extra latency hiding buys. The producer crosses unit boundaries, so
// a new unit's first chunks are already in flight while the previous unit
// finishes: the pipeline does not drain between units.
template <bool kWindow, bool kStream>
struct Producer {
  Work<kWindow, kStream> work;
  Unit U;
  int k;  // next chunk of U to issue
  bool done;
  // Cache pages and first slots of the two 16-key groups of chunk k, loaded
  // one chunk ahead so that the issue never waits for the block table.
  int32_t page[2];
  int32_t slot0[2];
  // Per-lane byte offsets within a 16-key group of one page (the cell view of
  // the cache): K and V of two key rows (one per 8-key half), and one scale.
  uint32_t off_k[2], off_v[2], off_s;
};

// The per-lane offsets of unit U's KV head.
template <class Prod>
__device__ __forceinline__ void producer_offsets(const AttnParams& p, Prod& P, int lane) {
  const uint32_t kq = lane >> 3, piece = lane & 7;
  const uint32_t head = static_cast<uint32_t>(P.U.kvh) * p.cell_head;
  const uint32_t sw = 16u * (piece ^ kq);  // row r's piece c goes to LDS position c ^ (r & 7)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t row = (8u * h + kq) * p.cell_slot + head + sw;
    P.off_k[h] = row + p.cell_off[0];
    P.off_v[h] = row + p.cell_off[1];
  }
  P.off_s = static_cast<uint32_t>(lane & 15) * p.cell_slot + head +
            (lane < 32 ? p.cell_off[2] : p.cell_off[3]);
}

// Block-table lookup for chunk k of the producer's unit (scalar loads; a
// 16-key group outside the unit's keys reads page 0 and is masked later).
template <class Prod>
__device__ __forceinline__ void producer_pages(const AttnParams& p, Prod& P) {
  const Unit& U = P.U;
  const int c = U.c_begin + kChunkTokens * P.k;
  const int64_t bt0 = static_cast<int64_t>(U.t.req) * p.bt_stride;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int c16 = c + 16 * sub;
    P.page[sub] = 0;
    P.slot0[sub] = 0;
    if (c16 < U.ld_hi && c16 + 16 > U.ld_lo) {
      const int blk = static_cast<int>(p.bs_div.div(c16));
      P.slot0[sub] = c16 - blk * static_cast<int>(p.bs_div.d);
      P.page[sub] = ld_ro(p.block_table, bt0 + blk);
    }
  }
}

// Moves the producer to its next chunk; false when the wave has no more.
template <class Prod>
__device__ __forceinline__ bool producer_next(const AttnParams& p, Prod& P, int lane) {
  while (!P.done && P.k >= P.U.n_chunks) {
    if (!P.work.next(p, lane, P.U)) {
      P.done = true;
      break;
    }
    P.k = 0;
    if (P.U.n_chunks > 0) {
      producer_offsets(p, P, lane);
      producer_pages(p, P);
    }
  }
  return !P.done;
}

// Issues the 9 direct-to-LDS loads of the producer's chunk k into `slot`:
// 4 x 1 KB of K, 4 x 1 KB of V (8 keys x 128 bytes each) and the 64 scales,
// then looks up the pages of chunk k + 1. Each 16-key group's address is a
// uniform 64-bit base (page * page stride + first slot * slot stride, on the
// scalar unit) plus the lane's 32-bit offset. Every address is inside the
// cache: a key outside the unit's range reads another slot of the same page
// (or of page 0) and is masked by the consumer, so every chunk issues
// exactly kDmaPerChunk loads.
template <class Prod>
__device__ __forceinline__ void issue_chunk(const AttnParams& p, Prod& P, char* slot, int lane) {
  const char* base[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    base[sub] = p.cell_base +
                static_cast<uint64_t>(static_cast<uint32_t>(P.page[sub])) * p.cell_block +
                static_cast<uint32_t>(P.slot0[sub]) * p.cell_slot;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dma16(base[i >> 1] + P.off_k[i & 1], slot + kSlotK + 1024 * i);
    dma16(base[i >> 1] + P.off_v[i & 1], slot + kSlotV + 1024 * i);
  }
  dma4(((lane >> 4) & 1 ? base[1] : base[0]) + P.off_s, slot + kSlotScale);
  ++P.k;
  if (P.k < P.U.n_chunks) producer_pages(p, P);
}

#ifndef PA_PAGED_WPE
#define PA_PAGED_WPE 2
#endif
template <bool kWindow, bool kStream, bool kF16Q, int kInFlight>
__global__ __launch_bounds__(kFwdWaves * 64) __attribute__((amdgpu_waves_per_eu(PA_PAGED_WPE, PA_PAGED_WPE)))
void attn_fwd_paged(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) char lds_all[kFwdWaves * kInFlight * kSlotBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char* lds = lds_all + wave * kInFlight * kSlotBytes;
  const uint32_t lds_base = lds_offset(lds);
  const ReadOffsets ro = read_offsets(lane);
  const float scl = scale_factor(lane & 15, p.scale_log2);

  Producer<kWindow, kStream> P;
  P.work.init(p, lane);
  P.U.n_chunks = 0;
  P.k = 0;
  P.done = false;
  Work<kWindow, kStream> work = P.work;  // the consumer's walk: the same units, behind
  Unit U;
  Lanes L;
  State st;
  bf16x8 qb[4], qlo[4];
  int ck = 0;
  bool have = false;
  int slot_r = 0;
  // The consumer's first unit is located, and its query load issued, before
  // the producer's first chunk: the two loads are in flight together (a
  // short launch is a chain of dependent loads per wave).
  while (work.next(p, lane, U)) {
    if (!U.has_rows) continue;
    L = unit_lanes<kWindow>(p, U, lane);
    if (U.n_chunks == 0) {  // no key of these rows in this split
      State empty;
      state_reset(empty);
      epilogue(p, U, L, empty);
      continue;
    }
    have = true;
    break;
  }
  if (have) load_q<kF16Q>(p, L, qb, qlo);

  int inflight = 0;  // chunks issued and not yet consumed
  int slot_w = 0;    // slot the producer fills next
#pragma unroll
  for (int i = 0; i < kInFlight; ++i) {
    if (producer_next(p, P, lane)) {
      issue_chunk(p, P, lds + slot_w * kSlotBytes, lane);
      ++inflight;
      slot_w = slot_w + 1 == kInFlight ? 0 : slot_w + 1;
    }
  }
  // Compiler-visible wait for the query (it also waits for the chunks just
  // issued, which the first step needs anyway).
  __builtin_amdgcn_s_waitcnt(0x0F70);
  state_reset(st);
  // The stores of a finished unit are issued after the wait that drains the
  // pipeline at the unit switch: vector memory operations complete in issue
  // order, so a store issued in front of chunks still in flight would make
  // every wait for those chunks wait for the store as well. The waits of
  // the chunks that were in flight before the stores count past them.
  int n_store = 0;
  int older_than_stores = 0;  // chunks in flight issued before the last stores
  while (true) {
    if (!have || ck >= U.n_chunks) {
      Finished done;
      const bool had = have;
      if (have) finish(U, L, st, done);
      have = false;
      while (work.next(p, lane, U)) {
        if (!U.has_rows) continue;
        L = unit_lanes<kWindow>(p, U, lane);
        if (U.n_chunks == 0) {  // no key of these rows in this split
          State empty;
          state_reset(empty);
          epilogue(p, U, L, empty);
          continue;
        }
        have = true;
        break;
      }
      if (have) load_q<kF16Q>(p, L, qb, qlo);
      // A compiler-visible wait for Q here (vmcnt(0): it also drains this
      // unit's chunks in flight, once per unit) keeps the compiler from
      // re-waiting for Q, with vmcnt(0), before every chunk of the loop.
      __builtin_amdgcn_s_waitcnt(0x0F70);
      if (had) {
        store_finished(p, done);
        n_store = stores_per_unit(p, done.s, done.live);
        older_than_stores = inflight;
      }
      if (!have) break;
      state_reset(st);
      ck = 0;
    }
    // Operations issued after the chunk about to be read: the next chunk's
    // loads when it is in flight, and the last unit's stores when they were
    // issued after this chunk's loads.
    wait_vmcnt_dyn((kInFlight >= 2 && inflight >= 2 ? kDmaPerChunk : 0) +
                   (older_than_stores > 0 ? n_store : 0));
    if (older_than_stores > 0) --older_than_stores;
    Chunk ch;
    read_chunk(lds_base + slot_r * kSlotBytes, ro, ch);  // returns once the reads landed
    --inflight;
    slot_r = slot_r + 1 == kInFlight ? 0 : slot_r + 1;
    if (producer_next(p, P, lane)) {
      issue_chunk(p, P, lds + slot_w * kSlotBytes, lane);
      ++inflight;
      slot_w = slot_w + 1 == kInFlight ? 0 : slot_w + 1;
    }
    compute_chunk<kF16Q>(U, L, U.c_begin + kChunkTokens * ck, ch, qb, qlo, scl, st);
    // Re-align the work-group's waves now and then: they read adjacent cells
    // whose shared cache lines are fetched once only while the waves stay
    // close (a wave running far ahead gets them evicted before its
    // neighbour asks). Only a rendezvous: no data passes through it, and a
    // wave that has finished its work no longer holds the others.
    if ((ck & (kRealignChunks - 1)) == kRealignChunks - 1) __builtin_amdgcn_s_barrier();
    ++ck;
  }
}

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
  const int64_t bt0 = static_cast<int64_t>(U.t.req) * p.bt_stride;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int c16 = c + 16 * sub;
    R.page[sub] = 0;
    R.slot0[sub] = 0;
    if (c16 < U.ld_hi && c16 + 16 > U.ld_lo) {
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
void attn_fwd_paged_reg(const AttnParams p) {
  const int lane = threadIdx.x & 63;
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
        if (PA_REG_REALIGN > 0 && (k % PA_REG_REALIGN) == PA_REG_REALIGN - 1) __builtin_amdgcn_s_barrier();
        if (++k >= U.n_chunks) break;
        if (k + 1 < U.n_chunks) {
          reg_load(p, R, lane, ca);
          if (k + 2 < U.n_chunks) reg_pages(p, U, c + 3 * kChunkTokens, R);
        }
        compute_chunk<kF16Q>(U, L, c + kChunkTokens, cb, qb, qlo, scl, st);
        if (PA_REG_REALIGN > 0 && (k % PA_REG_REALIGN) == PA_REG_REALIGN - 1) __builtin_amdgcn_s_barrier();
        if (++k >= U.n_chunks) break;
      }
    }
    epilogue(p, U, L, st);
  }
}

// Chunks in flight per wave on the paged path (LDS slots per wave).
constexpr int kPagedInFlight = PA_PAGED_INFLIGHT;

// Windows up to this many keys: the register-load kernel (its short
// latency wins when every row reads few keys); otherwise the direct-to-LDS
// pipeline (the higher sustained bandwidth on long rows).
constexpr int kShortWindow = 4096;

#ifndef PA_USE_STAGED
#define PA_USE_STAGED 1
#endif
template <bool W, bool St, bool F>
hipError_t launch_paged(const AttnParams& p, dim3 grid, hipStream_t stream) {
  if (PA_USE_STAGED && !(W && p.window > 0 && p.window <= kShortWindow))
    return launch_staged_kernel(p, grid, W, F, stream);
  if (PA_DECODE_REG || (W && p.window > 0 && p.window <= kShortWindow)) {
    hipLaunchKernelGGL((attn_fwd_paged_reg<W, St, F>), grid, dim3(kFwdWaves * 64), 0, stream, p);
  } else {
    hipLaunchKernelGGL((attn_fwd_paged<W, St, F, kPagedInFlight>), grid, dim3(kFwdWaves * 64), 0,
                       stream, p);
  }
  return hipGetLastError();
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
