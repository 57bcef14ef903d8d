// attn_device.h -- device building blocks shared by the attention kernels
// (attn_fwd.hip: the per-wave unit kernels; attn_rows.hip: the row-block
// kernel): operand types, int8 -> bf16 conversion, the 16x16x32 MFMA, row
// reductions, the LDS chunk slot and its direct-to-LDS loads, the per-lane
// row view, the online-softmax step of one 32-key chunk and the stores of a
// finished row group. The MFMA layout and the numerics are described at the
// top of attn_fwd.hip.

#pragma once

#include "attn_stream.h"

namespace pa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 4-byte-aligned vector loads: gfx950 runs dword-aligned multi-dword global
// accesses at full rate, and the vLLM cell only guarantees 4-byte (V) and
// 8-byte (K) alignment of a row.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float i8_to_f32(uint32_t w, int byte) {
  return static_cast<float>(static_cast<int32_t>(
      static_cast<int8_t>(static_cast<uint8_t>(w >> (8 * byte)))));
}

__device__ __forceinline__ bf16x2 pack_bf16(float a, float b) {
  return __builtin_convertvector((f32x2){a, b}, bf16x2);
}

// Eight int8 (two dwords, byte order) -> eight bf16.
__device__ __forceinline__ bf16x8 i8x8_to_bf16(uint32_t w0, uint32_t w1) {
  const bf16x2 p0 = pack_bf16(i8_to_f32(w0, 0), i8_to_f32(w0, 1));
  const bf16x2 p1 = pack_bf16(i8_to_f32(w0, 2), i8_to_f32(w0, 3));
  const bf16x2 p2 = pack_bf16(i8_to_f32(w1, 0), i8_to_f32(w1, 1));
  const bf16x2 p3 = pack_bf16(i8_to_f32(w1, 2), i8_to_f32(w1, 3));
  return (bf16x8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Byte `j` (0..7) of each of eight 8-byte runs -> eight bf16.
__device__ __forceinline__ bf16x8 column_to_bf16(const u32x2 (&v)[8], int j) {
  const int w = j >> 2, b = j & 3;
  bf16x2 p[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    p[e] = pack_bf16(i8_to_f32(v[2 * e][w], b), i8_to_f32(v[2 * e + 1][w], b));
  return (bf16x8){p[0][0], p[0][1], p[1][0], p[1][1],
                  p[2][0], p[2][1], p[3][0], p[3][1]};
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Reductions over the 4 lanes of a query row (lanes r, r + 16, r + 32,
// r + 48) with the gfx950 cross-row swaps. With both operands holding x,
// permlane16_swap returns {x of rows 0, 0, 2, 2 ; x of rows 1, 1, 3, 3} and
// permlane32_swap {x of the low half twice ; x of the high half twice}, so
// combining the pair gives the xor-16 (xor-32) partner's value; both lanes
// of a pair combine the same two values in the same order, so all 4 lanes
// end with the same result. The two results are copied to named scalars
// before use: indexing the returned pair inside a bit cast reads element 0
// twice with this compiler.
struct SwapPair {
  float a, b;
};
__device__ __forceinline__ SwapPair swap_rows16(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return {__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1)};
}
__device__ __forceinline__ SwapPair swap_halves(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return {__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1)};
}
// max of two floats as the bare instruction: fmaxf would first quiet the
// operands that come from a cross-lane move (2 extra instructions each).
__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Max of a lane's 8 scores (finite or -inf, never NaN) in 4 instructions.
__device__ __forceinline__ float max8_raw(const float (&t)[8]) {
  return max3_raw(max3_raw(t[0], t[1], t[2]), max3_raw(t[3], t[4], t[5]), max_raw(t[6], t[7]));
}
__device__ __forceinline__ float xor_max(float x) {
  const SwapPair a = swap_rows16(x);
  const SwapPair b = swap_halves(max_raw(a.a, a.b));
  return max_raw(b.a, b.b);
}
__device__ __forceinline__ float xor_sum(float x) {
  const SwapPair a = swap_rows16(x);
  const SwapPair b = swap_halves(a.a + a.b);
  return b.a + b.b;
}

// The cache bytes of one 32-key chunk for one lane.
struct Chunk {
  u32x4 k[2][2];  // K: 32 bytes of key (16 sub + r) for sub = 0, 1
  u32x2 v[8];     // V: 8 bytes of key tv(e)
  float sc;       // one scale: see load_chunk
};

// Lane n of every 16-lane row, broadcast to the row (DPP row_newbcast).
// Waves per work-group of the attention kernel: one per KV head of a decode
// tile, so the 8 cells of a token (8 x 264 contiguous bytes for NHD pages)
// are read by one CU.
constexpr int kFwdWaves = kGroupUnits;
// LDS staging of the paged path: two 32-key chunk slots per wave, each
// [K: 32 x 128 B | V: 32 x 128 B | k_scale x 32, v_scale x 32].
constexpr int kSlotK = 0;
constexpr int kSlotV = 4096;
constexpr int kSlotScale = 8192;
constexpr int kSlotBytes = 8192 + 256;
// Direct-to-LDS loads of one chunk: 4 for K, 4 for V, 1 for the scales.
constexpr int kDmaPerChunk = 9;
// Chunks between the waves' rendezvous in the paged kernel. Adjacent heads'
// cells share cache lines (a 264-byte cell is not line-aligned); the closer
// the waves stay, the fewer of those lines are fetched twice. Measured on 64
// sequences of 1k-32k keys: every chunk fetches only the algorithmic bytes
// but idles waves at the barrier; every 32 fetches 10 % more; 8 is fastest.
constexpr int kRealignChunks = 8;

// s_waitcnt with only the vector-memory counter (<= n outstanding) or only
// the LDS counter (0 outstanding). Inline asm with a memory clobber, so the
// compiler neither moves memory operations across it nor drops it: the
// direct-to-LDS loads are not tracked against later LDS reads by the
// compiler's own wait insertion.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// One 16-byte (or 4-byte) global -> LDS copy per lane: lane i's bytes land at
// lds + 16 i (4 i). `lds` must be wave-uniform.
__device__ __forceinline__ void dma16(const char* g, char* lds) {
  __builtin_amdgcn_global_load_lds(
      (const void __attribute__((address_space(1)))*)(g),
      (void __attribute__((address_space(3)))*)(lds), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const char* g, char* lds) {
  __builtin_amdgcn_global_load_lds(
      (const void __attribute__((address_space(1)))*)(g),
      (void __attribute__((address_space(3)))*)(lds), 4, 0, 0);
}
// A global load with the non-temporal hint (cache policy nt): for cache
// bytes that the launch reads once and no other wave reads.
template <class T>
__device__ __forceinline__ T ld_nt(const char* g) {
  return __builtin_nontemporal_load(reinterpret_cast<const T*>(g));
}

// K/V rows in a slot are 128 bytes; their 16-byte pieces are stored in the
// order piece ^ (key & 7), so the reads below (8 keys at the same piece per
// 8 lanes for K, one key per 16 lanes for V) touch distinct banks.
__device__ __forceinline__ int swz(int key, int piece) { return 128 * key + 16 * (piece ^ (key & 7)); }

template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x),
                                                            0x150 + N, 0xf, 0xf, false));
}

// The chunk's 8 K scales (times scale * log2 e) and 8 V scales of a lane,
// from sc1 = (the lane's slot scale) * (scale * log2 e for K lanes, 1 for V):
// lane r16 < 8 of a row holds the K scale of key 16 (r16 / 4) + 4 g + r16 % 4,
// lane 8 + e the V scale of the same key.
__device__ __forceinline__ void lane_scales(float sc1, float (&ks)[8], float (&vs)[8]) {
  ks[0] = row_bcast<0>(sc1);
  ks[1] = row_bcast<1>(sc1);
  ks[2] = row_bcast<2>(sc1);
  ks[3] = row_bcast<3>(sc1);
  ks[4] = row_bcast<4>(sc1);
  ks[5] = row_bcast<5>(sc1);
  ks[6] = row_bcast<6>(sc1);
  ks[7] = row_bcast<7>(sc1);
  vs[0] = row_bcast<8>(sc1);
  vs[1] = row_bcast<9>(sc1);
  vs[2] = row_bcast<10>(sc1);
  vs[3] = row_bcast<11>(sc1);
  vs[4] = row_bcast<12>(sc1);
  vs[5] = row_bcast<13>(sc1);
  vs[6] = row_bcast<14>(sc1);
  vs[7] = row_bcast<15>(sc1);
}

__device__ __forceinline__ const char* at(const CacheStream& s, int64_t page,
                                          int32_t slot, int32_t head) {
  return s.base + page * s.s_block + static_cast<int64_t>(slot) * s.s_slot +
         static_cast<int64_t>(head) * s.s_head;
}

// Everything about one work unit that is uniform across the wave: rows
// [16 rg, 16 rg + 16) of row tile t, KV head kvh, the keys [c_lo, c_hi) of
// split s of the row tile's stream (live splits in all).
struct Unit {
  RowTile t;
  int s, live, kvh, rg;
  int rows;      // query rows of the row tile (num_tok * G)
  int row0;      // first row of this wave (16 rg)
  bool has_rows;  // row0 < rows
  int ld_lo, ld_hi;  // keys the wave reads: [ld_lo, ld_hi)
  int c_begin;       // first chunk (32-aligned)
  int n_chunks;
  int w_lo_max, w_hi_min;  // a chunk outside [w_lo_max, w_hi_min] needs the mask
};

// Unit of KV-head unit hu (= kvh * row groups + rg) of row tile t over the
// keys [c_lo, c_hi) (c_lo 32-aligned), trimmed to the keys its rows see.
template <bool kWindow>
__device__ __forceinline__ void make_unit(const AttnParams& p, const RowTile& t, int hu,
                                          int c_lo, int c_hi, int s, int live, Unit& U) {
  const int window = kWindow ? p.window : 0;
  const bool causal = kWindow ? (p.causal != 0) : true;
  U.t = t;
  U.s = s;
  U.live = live;
  U.kvh = static_cast<int>(p.rg_div.div(hu));
  U.rg = hu - U.kvh * static_cast<int>(p.rg_div.d);
  const int G = p.group;
  U.rows = U.t.num_tok * G;
  U.row0 = U.rg * kRowsPerWave;
  U.has_rows = U.row0 < U.rows;
  U.n_chunks = 0;
  if (!U.has_rows) return;
  const int wrow_end = U.row0 + kRowsPerWave < U.rows ? U.row0 + kRowsPerWave : U.rows;
  const int tok_first = U.t.tok_begin + static_cast<int>(p.g_div.div(U.row0));
  const int tok_last = U.t.tok_begin + static_cast<int>(p.g_div.div(wrow_end - 1));
  const int w_lo_min = key_lo(U.t, tok_first, window);
  U.w_lo_max = key_lo(U.t, tok_last, window);
  U.w_hi_min = key_hi(U.t, tok_first, window, causal);
  const int w_hi_max = key_hi(U.t, tok_last, window, causal);
  U.ld_lo = c_lo > w_lo_min ? c_lo : w_lo_min;
  U.ld_hi = c_hi < w_hi_max + 1 ? c_hi : w_hi_max + 1;
  U.c_begin = U.ld_lo & ~(kChunkTokens - 1);
  U.n_chunks = U.c_begin < U.ld_hi ? (U.ld_hi - U.c_begin + kChunkTokens - 1) / kChunkTokens : 0;
}

// The work of one wave, in the order it runs it. Two partitions:
//   * num_splits == 1: units are (request, row tile, KV-head unit), whole
//     key ranges; wave w of the grid's W waves takes units w, w + W, ...,
//     of a table derived on the device from query_start_loc and seq_lens
//     (a prefix sum over requests, 64 per wave instruction).
//   * num_splits > 1 (kStream): the chunk-stream partition of
//     attn_geometry.h. Work-group b runs positions [b per, (b + 1) per);
//     wave w of it takes KV-head unit 8 g + w of each group g it meets, so
//     the 8 waves of a work-group read the 8 adjacent heads of the same keys
//     (their cells share cache lines), and every split but a stream's last
//     is exactly per chunks long.
template <bool kWindow, bool kStream>
struct Work {
  // num_splits == 1
  int r0 = -64;  // first request of the cursor's 64-request window
  int u0 = 0;    // units before the window
  int u1 = 0;    // units through the window
  int incl = 0;  // per lane: inclusive prefix within the window
  int next_u = 0;
  int stride = 0;
  // num_splits > 1
  StreamCursor sc;
  StreamDesc d;
  int64_t pos = 0, stop = 0, per = 1;
  int wg = 0, wave = 0;

  // kPrime: size the partition and load the first cursor window with the
  // same loads (stream_per_cursor). Off for the page-row kernel, whose
  // launches are long enough that the round trip does not show and whose
  // chunk loop ran ~0.5 % slower with the primed cursor's code.
  template <bool kPrime = true>
  __device__ __forceinline__ void init(const AttnParams& p, int lane) {
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    if constexpr (kStream) {
      // kGroupUnits / gu partition work-groups per work-group, interleaved:
      // waves [v gu, (v + 1) gu) of work-group b are partition work-group
      // v W + b (W work-groups), so a launch with little work still spreads
      // its first partition work-groups over W compute units.
      const int vpw = kGroupUnits / p.gu;
      d = StreamDesc{p.qsl, p.seq_lens, p.num_reqs, p.bq, kWindow ? p.window : 0,
                     kWindow ? p.causal : 1, p.n_hg, static_cast<int32_t>(gridDim.x) * vpw,
                     p.num_splits};
      int64_t total;
      if constexpr (kPrime) per = stream_per_cursor(d, lane, total, sc);
      else per = stream_per(d, lane, total);
      wg = (w / p.gu) * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x);
      wave = w % p.gu;
      pos = static_cast<int64_t>(wg) * per + kStreamStartPositions;
      stop = pos + per < total ? pos + per : total;
    } else {
      next_u = blockIdx.x * kGroupUnits + w;
      stride = gridDim.x * kGroupUnits;
    }
  }

  // The next unit of this wave (possibly without rows or keys); false at the
  // end of its work.
  __device__ __forceinline__ bool next(const AttnParams& p, int lane, Unit& U) {
    if constexpr (kStream) {
      while (pos < stop) {
        StreamPos sp;
        if (!stream_locate(d, sc, pos, lane, sp)) {
          pos = stop;
          return false;
        }
        // The work-group's chunks of this stream: [c0, c1). A range that
        // holds only the stream's start positions has none (the next
        // work-group starts the stream).
        const int64_t cs = sp.c0 + kStreamStartPositions;
        const int c0 = pos > cs ? static_cast<int>(pos - cs) : 0;
        const int64_t end = cs + sp.n < stop ? cs + sp.n : stop;
        const int c1 = static_cast<int>(end - cs);
        pos = end;
        if (c1 <= c0) continue;
        const int hu = sp.hg * p.gu + wave;
        if (hu >= p.n_hu) continue;  // the group has fewer units than waves
        int first, live;
        stream_splits(sp.c0, sp.n, per, first, live);
        make_unit<kWindow>(p, sp.t, hu, sp.cb + kChunkTokens * c0, sp.cb + kChunkTokens * c1,
                           wg - first, live, U);
        return true;
      }
      return false;
    } else {
      const int window = kWindow ? p.window : 0;
      const bool causal = kWindow ? (p.causal != 0) : true;
      const int u = next_u;
      next_u += stride;
      while (u >= u1) {
        r0 += 64;
        u0 = u1;
        if (r0 >= p.num_reqs) return false;
        const int r = r0 + lane;
        const int units =
            r < p.num_reqs ? request_row_tiles(p.qsl[r + 1] - p.qsl[r], p.bq) * p.n_hu : 0;
        const int x = wave_scan32(units);
        incl = x;
        u1 = u0 + __builtin_amdgcn_readlane(x, 63);
      }
      const int local = u - u0;
      const int j = static_cast<int>(__popcll(__ballot(incl <= local)));
      const int req = r0 + j;
      const int u_loc = local - (j > 0 ? __builtin_amdgcn_readlane(incl, j - 1) : 0);
      const int q_start = ld_ro(p.qsl, req);
      const int q_len = ld_ro(p.qsl, req + 1) - q_start;
      const int seq_len = ld_ro(p.seq_lens, req);
      const RowTile t = request_tile(req, q_start, q_len, seq_len, p.bq, u_loc / p.n_hu);
      make_unit<kWindow>(p, t, u_loc % p.n_hu, tile_chunk_base(t, window),
                         range_end(t, window, causal), 0, 1, U);
      return true;
    }
  }
};

// Per-lane view of the unit's rows: lane l holds row row0 + (l % 16).
struct Lanes {
  int r16, g;
  bool vrow;
  int head;
  int64_t qtok;
  int lo, hi;
};

// The one scale a lane holds for a chunk (see read_chunk): the K scales of
// lanes r < 8 are pre-multiplied by softmax_scale * log2(e) before the row
// broadcast.
__device__ __forceinline__ float scale_factor(int r16, float scale_log2) {
  return r16 < 8 ? scale_log2 : 1.0f;
}

template <bool kWindow>
__device__ __forceinline__ Lanes unit_lanes(const AttnParams& p, const Unit& U, int lane) {
  const int window = kWindow ? p.window : 0;
  const bool causal = kWindow ? (p.causal != 0) : true;
  Lanes L;
  L.r16 = lane & 15;
  L.g = lane >> 4;
  const int row = U.row0 + L.r16;
  L.vrow = row < U.rows;
  const int rr = L.vrow ? row : U.row0;
  const int tok = static_cast<int>(p.g_div.div(static_cast<uint32_t>(rr)));
  L.head = U.kvh * p.group + (rr - tok * p.group);
  L.qtok = static_cast<int64_t>(U.t.q_start) + U.t.tok_begin + tok;
  L.lo = key_lo(U.t, U.t.tok_begin + tok, window);
  L.hi = key_hi(U.t, U.t.tok_begin + tok, window, causal);
  return L;
}

// Head-size geometry of the per-lane layout (the comment at the top of
// attn_fwd.hip describes D = 128). Lane (r, g) holds, per key, bytes
// [g D/4, (g + 1) D/4) of K (QK MFMA j takes bytes 8j .. 8j + 8 of them);
// per V run, bytes [r D/16, (r + 1) D/16) of 8 keys (PV MFMA j takes byte
// j); and O[row][(D/16)(4g + i) + j] in o[j][i], i.e. the D/4 contiguous
// output columns [g D/4, (g + 1) D/4).
template <int D>
struct HeadDim {
  static_assert(D == 64 || D == 128 || D == 256, "head size 64, 128 or 256");
  static constexpr int kQK = D / 32;  // QK MFMAs per 16 keys (Q operands per lane)
  static constexpr int kPV = D / 16;  // PV MFMAs (output column groups)
  static constexpr int kCols = D / 4; // output columns per lane
};

// Q^T as the B operand of QK: qb[j] holds Q[row][g D/4 + 8 j .. + 8] in bf16
// (and, for an fp16 q, qlo[j] the exact remainder q - bf16(q)). load_q_raw
// issues the 16-byte loads; q_operands converts them.
template <int D = 128>
__device__ __forceinline__ void load_q_raw(const AttnParams& p, const Lanes& L,
                                           u32x4 (&raw)[HeadDim<D>::kQK]) {
  const char* qrow = p.q + L.qtok * p.s_q_tok + static_cast<int64_t>(L.head) * p.s_q_head;
#pragma unroll
  for (int j = 0; j < HeadDim<D>::kQK; ++j)
    raw[j] = L.vrow ? *reinterpret_cast<const u32x4*>(qrow + 2 * (HeadDim<D>::kCols * L.g + 8 * j))
                    : (u32x4){0u, 0u, 0u, 0u};
}

template <bool kF16Q, int N>
__device__ __forceinline__ void q_operands(const u32x4 (&raw)[N], bf16x8 (&qb)[N],
                                           bf16x8 (&qlo)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    if constexpr (kF16Q) {
      // fp16 q = hi + lo with hi = bf16(q), lo = bf16(q - hi): exact, since an
      // fp16 significand has 11 bits and each bf16 holds 8.
      const f16x8 h = __builtin_bit_cast(f16x8, raw[j]);
      bf16x8 a, b;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = static_cast<float>(h[e]);
        const __bf16 fh = static_cast<__bf16>(f);
        a[e] = fh;
        b[e] = static_cast<__bf16>(f - static_cast<float>(fh));
      }
      qb[j] = a;
      qlo[j] = b;
    } else {
      qb[j] = __builtin_bit_cast(bf16x8, raw[j]);
      qlo[j] = qb[j];
    }
  }
}

template <bool kF16Q, int D = 128>
__device__ __forceinline__ void load_q(const AttnParams& p, const Lanes& L,
                                       bf16x8 (&qb)[HeadDim<D>::kQK],
                                       bf16x8 (&qlo)[HeadDim<D>::kQK]) {
  u32x4 raw[HeadDim<D>::kQK];
  load_q_raw<D>(p, L, raw);
  q_operands<kF16Q>(raw, qb, qlo);
}

// Online-softmax state of one wave's 16 rows.
template <int D>
struct StateT {
  f32x4 o[HeadDim<D>::kPV];  // o[j][i] = O[row][(D/16)(4g + i) + j] (unnormalised)
  float m;                   // running max (log2 units), equal in the 4 lanes of a row
  float l;                   // this lane's part of the running sum
};
using State = StateT<128>;

template <int D>
__device__ __forceinline__ void state_reset(StateT<D>& st) {
#pragma unroll
  for (int j = 0; j < HeadDim<D>::kPV; ++j) st.o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  st.m = kNegInf;
  st.l = 0.0f;
}

// One 32-key chunk starting at key c: S = K Q^T, mask, online softmax, O += V P.
// The reference max m only moves when a row's chunk max exceeds it by more
// than kRescaleSlack (log2 units): p = 2^(s - m) then stays <= 2^8, exact
// in fp32 accumulation and bf16 hi + lo, and the O rescale is skipped for
// every chunk where no row's max grew that much (all chunks but a few at
// the start of a long row). The result is the same softmax: the final
// normalisation divides the common factor out. A row's first chunk with a
// visible key always sets m.
constexpr float kRescaleSlack = 8.0f;

// A row's m moves when its chunk max exceeds this: kRescaleSlack, or for a
// row with no visible key yet (m = -inf) any visible score (a score is
// finite, so > -FLT_MAX is the same test as > -inf; one compare either way).
__device__ __forceinline__ float rescale_threshold(bool fresh) {
  return fresh ? -3.402823466e38f : kRescaleSlack;
}

// The operands of a chunk in registers as the D = 128 paged kernels load
// them (Chunk); ops.k(sub, j) / ops.v(j) give the bf16 K and V operands and
// ops.sc the lane's scale.
struct ChunkOps {
  const Chunk& ch;
  __device__ __forceinline__ float sc() const { return ch.sc; }
  __device__ __forceinline__ bf16x8 k(int sub, int j) const {
    const u32x4& w = ch.k[sub][j >> 1];
    return (j & 1) ? i8x8_to_bf16(w[2], w[3]) : i8x8_to_bf16(w[0], w[1]);
  }
  __device__ __forceinline__ bf16x8 v(int j) const { return column_to_bf16(ch.v, j); }
};

// The rest of a chunk step after QK: t = the lane's 8 scores minus m_use (log2
// units), vs its V scales.
template <int D, class Ops>
__device__ __forceinline__ void chunk_tail(const Unit& U, const Lanes& L, int c, const Ops& ops,
                                           float (&t)[8], float (&vs)[8], bool fresh, float m_use,
                                           StateT<D>& st);

template <int D, bool kF16Q, class Ops>
__device__ __forceinline__ void compute_chunk_t(const Unit& U, const Lanes& L, int c,
                                                const Ops& ops,
                                                const bf16x8 (&qb)[HeadDim<D>::kQK],
                                                const bf16x8 (&qlo)[HeadDim<D>::kQK], float scl,
                                                StateT<D>& st) {
  const float sc1 = ops.sc() * scl;
  const float ks[8] = {row_bcast<0>(sc1), row_bcast<1>(sc1), row_bcast<2>(sc1),
                       row_bcast<3>(sc1), row_bcast<4>(sc1), row_bcast<5>(sc1),
                       row_bcast<6>(sc1), row_bcast<7>(sc1)};
  float vs[8] = {row_bcast<8>(sc1),  row_bcast<9>(sc1),  row_bcast<10>(sc1),
                 row_bcast<11>(sc1), row_bcast<12>(sc1), row_bcast<13>(sc1),
                 row_bcast<14>(sc1), row_bcast<15>(sc1)};
  const bool fresh = st.m == kNegInf;
  const float m_use = fresh ? 0.0f : st.m;
  float t[8];  // score - m_use (log2 units)
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < HeadDim<D>::kQK; ++j) {
      const bf16x8 a = ops.k(sub, j);
      acc = mfma(a, qb[j], acc);
      if constexpr (kF16Q) acc = mfma(a, qlo[j], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) t[4 * sub + i] = fmaf(acc[i], ks[4 * sub + i], -m_use);
  }
  chunk_tail<D>(U, L, c, ops, t, vs, fresh, m_use, st);
}

template <int D, class Ops>
__device__ __forceinline__ void chunk_tail(const Unit& U, const Lanes& L, int c, const Ops& ops,
                                           float (&t)[8], float (&vs)[8], bool fresh, float m_use,
                                           StateT<D>& st) {
  if (c < U.w_lo_max || c + kChunkTokens - 1 > U.w_hi_min) {
    // A key outside the row's range (or the request) gets p = 0 and a zero
    // V scale: its cache bytes may be any bits, a scale included.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = c + 16 * (e >> 2) + 4 * L.g + (e & 3);
      if (key < L.lo || key > L.hi) {
        t[e] = kNegInf;
        vs[e] = 0.0f;
      }
    }
  }
  // A row's max exceeds the threshold iff one of its 4 lanes' maxima does:
  // the cross-lane reduction runs only when some row grows (rarely, past the
  // first chunks).
  const float lane_mx = max8_raw(t);
  if (__ballot(lane_mx > rescale_threshold(fresh)) != 0) {
    const float mx = xor_max(lane_mx);
    const bool grow = mx > rescale_threshold(fresh);
    // Rows that keep m (also rows with no visible key yet) scale by 1.
    const float alpha = grow && !fresh ? __builtin_amdgcn_exp2f(-mx) : 1.0f;
    st.l *= alpha;
#pragma unroll
    for (int j = 0; j < HeadDim<D>::kPV; ++j) st.o[j] *= alpha;
    const float shift = grow ? mx : 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] -= shift;
    st.m = grow ? m_use + mx : st.m;
  }
  float pv[8];
  float lsum;  // the sum starts at the first term (an added 0 is an instruction)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pe = __builtin_amdgcn_exp2f(t[e]);
    lsum = e == 0 ? pe : lsum + pe;
    pv[e] = pe * vs[e];
  }
  st.l += lsum;
  // P = hi + lo in bf16 (16 significant bits together): a single bf16 P would
  // carry a 2^-9 relative error into the output whenever the softmax is
  // peaked (short contexts, early causal rows).
  bf16x8 p_hi, p_lo;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bf16x2 h = pack_bf16(pv[e], pv[e + 1]);
    const uint32_t hb = __builtin_bit_cast(uint32_t, h);
    const float h0 = __builtin_bit_cast(float, hb << 16);
    const float h1 = __builtin_bit_cast(float, hb & 0xffff0000u);
    const bf16x2 lw = pack_bf16(pv[e] - h0, pv[e + 1] - h1);
    p_hi[e] = h[0];
    p_hi[e + 1] = h[1];
    p_lo[e] = lw[0];
    p_lo[e + 1] = lw[1];
  }
#pragma unroll
  for (int j = 0; j < HeadDim<D>::kPV; ++j) {
    const bf16x8 vcol = ops.v(j);
    st.o[j] = mfma(vcol, p_hi, st.o[j]);
    st.o[j] = mfma(vcol, p_lo, st.o[j]);
  }
}

template <bool kF16Q>
__device__ __forceinline__ void compute_chunk(const Unit& U, const Lanes& L, int c,
                                              const Chunk& ch, const bf16x8 (&qb)[4],
                                              const bf16x8 (&qlo)[4], float scl,
                                              State& st) {
  compute_chunk_t<128, kF16Q>(U, L, c, ChunkOps{ch}, qb, qlo, scl, st);
}

// ---------------------------------------------------------------------------
// Integer QK for the D = 128 paged kernels. The K bytes of a chunk are the A
// operand of v_mfma_i32_16x16x64_i8 as they are loaded (lane (r, g) holds
// bytes [32 g + 16 h, 32 g + 16 h + 16) of key r for product h = 0, 1), so K
// is never converted; the B side maps its bytes to the same columns, so a
// product sums over all 128 columns whatever order the hardware reduces in.
// Each query row is scaled by 2^S (S from the row's largest |q|) and rounded
// to integers x with |x| < 2^20, written as three digits
// x = d0 2^14 + d1 2^7 + d2 (d0 = x >> 14 in [-64, 63], d1, d2 in [0, 127]),
// and each digit is the B operand of one integer product. The products are
// exact in int32; the score is (2^14 acc0 + (2^7 acc1 + acc2)) 2^-S, the
// inner sum exact in int32 and one fp32 fma joining it to 2^14 acc0 (with
// 2^-S applied by the lane, whose row is fixed). A query element within
// 2^-13 (bf16) or 2^-10 (fp16) of its row's largest in binary order of
// magnitude is exact; a smaller one is rounded to 2^-20 of the row's largest,
// below the fp32 rounding of the score. A non-finite query element makes its
// row's scores NaN.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

struct QInt8 {
  i32x4 d[3][2];  // [digit][h]: digits of the lane's 16 query bytes of product h
  float r;        // 2^-S of the lane's row (NaN for a row with a non-finite element)
  float r14;      // 2^14 r
};

template <bool kF16Q>
__device__ __forceinline__ void load_q_int8(const AttnParams& p, const Lanes& L, QInt8& q) {
  u32x4 raw[4];
  load_q_raw<128>(p, L, raw);
  float f[32];  // raw[j] element e: query column 32 g + 8 j + e
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (kF16Q) {
      const f16x8 h = __builtin_bit_cast(f16x8, raw[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[8 * j + e] = static_cast<float>(h[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = raw[j][e >> 1];
        f[8 * j + e] = __builtin_bit_cast(float, (e & 1) ? (w & 0xffff0000u) : (w << 16));
      }
    }
  }
  float amax = 0.0f, bad = 0.0f;  // bad: 1 for an element that is inf or NaN
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    amax = fmaxf(amax, fabsf(f[e]));
    bad = fabsf(f[e]) <= 3.402823466e38f ? bad : 1.0f;
  }
  amax = xor_max(amax);  // over the 4 lanes of the row
  bad = xor_max(bad);
  // amax < 2^E with E the exponent field - 126 (clamped so that 2^-S stays a
  // normal float); S = 20 - E gives |q| 2^S < 2^20.
  int E = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xff) - 126;
  E = E < -100 ? -100 : (E > 128 ? 128 : E);
  const int S = 20 - E;
  q.r = bad == 0.0f ? __builtin_ldexpf(1.0f, -S) : __builtin_nanf("");
  q.r14 = 16384.0f * q.r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // product h, byte 4 w + i: column 32 g + 16 h + 4 w + i = f[16 h + 4 w + i]
        const float v = bad == 0.0f ? f[16 * h + 4 * w + i] : 0.0f;
        const int x = static_cast<int>(__builtin_rintf(__builtin_ldexpf(v, S)));
        b0 |= (static_cast<uint32_t>(x >> 14) & 0xffu) << (8 * i);
        b1 |= (static_cast<uint32_t>(x >> 7) & 0x7fu) << (8 * i);
        b2 |= (static_cast<uint32_t>(x) & 0x7fu) << (8 * i);
      }
      q.d[0][h][w] = static_cast<int32_t>(b0);
      q.d[1][h][w] = static_cast<int32_t>(b1);
      q.d[2][h][w] = static_cast<int32_t>(b2);
    }
  }
}

__device__ __forceinline__ i32x4 mfma_i8(const u32x4& a, const i32x4& b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), b, c, 0, 0, 0);
}

__device__ __forceinline__ void compute_chunk(const Unit& U, const Lanes& L, int c,
                                              const Chunk& ch, const QInt8& q, float scl,
                                              State& st) {
  const ChunkOps ops{ch};
  const float sc1 = ops.sc() * scl;
  const float ks[8] = {row_bcast<0>(sc1), row_bcast<1>(sc1), row_bcast<2>(sc1),
                       row_bcast<3>(sc1), row_bcast<4>(sc1), row_bcast<5>(sc1),
                       row_bcast<6>(sc1), row_bcast<7>(sc1)};
  float vs[8] = {row_bcast<8>(sc1),  row_bcast<9>(sc1),  row_bcast<10>(sc1),
                 row_bcast<11>(sc1), row_bcast<12>(sc1), row_bcast<13>(sc1),
                 row_bcast<14>(sc1), row_bcast<15>(sc1)};
  const bool fresh = st.m == kNegInf;
  const float m_use = fresh ? 0.0f : st.m;
  float t[8];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    i32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      a0 = mfma_i8(ch.k[sub][h], q.d[0][h], a0);
      a1 = mfma_i8(ch.k[sub][h], q.d[1][h], a1);
      a2 = mfma_i8(ch.k[sub][h], q.d[2][h], a2);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sc = fmaf(static_cast<float>(a0[i]), q.r14,
                            static_cast<float>(a1[i] * 128 + a2[i]) * q.r);
      t[4 * sub + i] = fmaf(sc, ks[4 * sub + i], -m_use);
    }
  }
  chunk_tail<128>(U, L, c, ops, t, vs, fresh, m_use, st);
}

// A finished unit's result, held in registers until it is stored.
template <int D>
struct FinishedT {
  float res[HeadDim<D>::kCols];  // res[(D/16) i + j] = normalised O[row][g D/4 + (D/16) i + j]
  float lse2;                    // log2-sum-exp of the row, -inf without a visible key
  int64_t qtok;
  int head, g;
  bool vrow;
  int s, live;
};
using Finished = FinishedT<128>;

template <int D>
__device__ __forceinline__ void finish(const Unit& U, const Lanes& L, const StateT<D>& st,
                                       FinishedT<D>& f) {
  constexpr int kPV = HeadDim<D>::kPV;
  const float l_tot = xor_sum(st.l);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
#pragma unroll
  for (int j = 0; j < kPV; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) f.res[kPV * i + j] = st.o[j][i] * inv;
  f.lse2 = l_tot > 0.0f ? st.m + __builtin_amdgcn_logf(l_tot) : kNegInf;
  f.qtok = L.qtok;
  f.head = L.head;
  f.g = L.g;
  f.vrow = L.vrow;
  f.s = U.s;
  f.live = U.live;
}

// Whether a finished unit goes to out (num_splits == 1, or a single-split
// stream when the launch writes those directly) or to the split partials.
__device__ __forceinline__ bool direct_out(const AttnParams& p, int live) {
  return p.num_splits == 1 || (live == 1 && p.direct_single != 0);
}

// Split count marker. On the op path (direct_single) the combine must know
// how many splits a row has. The unit that computes split 0 of a row with
// live < num_splits splits records live in the row's last log2-LSE slot,
// num_splits - 1, which no split of the row uses: as a quiet NaN whose
// payload is live (a real LSE is finite or -inf, and a NaN produced by
// arithmetic has payload 0). With live == num_splits no marker is written
// and the combine reads all splits.
constexpr uint32_t kSplitMarker = 0x7fc00000u;
__device__ __forceinline__ bool writes_marker(const AttnParams& p, int s, int live) {
  return p.direct_single != 0 && p.num_splits > 1 && s == 0 && live < p.num_splits;
}

// Stores a finished unit: out (and lse_out, natural log) or its split's
// partials. Split slots a row does not use are left untouched here
// (fill_unused_splits writes them when a caller needs them).
template <int D>
__device__ __forceinline__ void store_finished(const AttnParams& p, const FinishedT<D>& f) {
  constexpr int kCols = HeadDim<D>::kCols;
  if (!f.vrow) return;
  const int g = f.g;
  const int64_t head = f.head;
  if (writes_marker(p, f.s, f.live)) {
    char* lse_row = reinterpret_cast<char*>(p.ws_lse) + f.qtok * p.s_wl_tok + head * p.s_wl_head;
    *reinterpret_cast<uint32_t*>(lse_row + static_cast<int64_t>(p.num_splits - 1) * p.s_wl_split) =
        kSplitMarker | static_cast<uint32_t>(f.live);
  }
  if (!direct_out(p, f.live)) {
    char* dst = reinterpret_cast<char*>(p.ws_o) + f.s * p.s_wo_split + f.qtok * p.s_wo_tok +
                head * p.s_wo_head + 4 * kCols * g;
#pragma unroll
    for (int k = 0; k < kCols / 4; ++k)
      *reinterpret_cast<f32x4*>(dst + 16 * k) =
          (f32x4){f.res[4 * k], f.res[4 * k + 1], f.res[4 * k + 2], f.res[4 * k + 3]};
    // The 4 lanes of a row hold the same lse2 and store it to the same place.
    char* lse_row = reinterpret_cast<char*>(p.ws_lse) + f.qtok * p.s_wl_tok + head * p.s_wl_head;
    *reinterpret_cast<float*>(lse_row + f.s * p.s_wl_split) = f.lse2;
    return;
  }
  char* dst = p.out + f.qtok * p.s_out_tok + head * p.s_out_head;
  if (p.out_dtype == PTH_ATTN_BF16) {
    dst += 2 * kCols * g;
#pragma unroll
    for (int k = 0; k < kCols / 8; ++k) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf16x2 pr = pack_bf16(f.res[8 * k + e], f.res[8 * k + e + 1]);
        v[e] = pr[0];
        v[e + 1] = pr[1];
      }
      *reinterpret_cast<bf16x8*>(dst + 16 * k) = v;
    }
  } else if (p.out_dtype == PTH_ATTN_F16) {
    dst += 2 * kCols * g;
#pragma unroll
    for (int k = 0; k < kCols / 8; ++k) {
      f16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<_Float16>(f.res[8 * k + e]);
      *reinterpret_cast<f16x8*>(dst + 16 * k) = v;
    }
  } else {
    dst += 4 * kCols * g;
#pragma unroll
    for (int k = 0; k < kCols / 4; ++k)
      *reinterpret_cast<f32x4*>(dst + 16 * k) =
          (f32x4){f.res[4 * k], f.res[4 * k + 1], f.res[4 * k + 2], f.res[4 * k + 3]};
  }
  if (p.lse_out != nullptr) {
    float* lo_ptr = reinterpret_cast<float*>(reinterpret_cast<char*>(p.lse_out) +
                                             f.qtok * p.s_lo_tok + head * p.s_lo_head);
    *lo_ptr = f.lse2 * 0.69314718055994530942f;
  }
}

template <int D>
__device__ __forceinline__ void epilogue(const AttnParams& p, const Unit& U, const Lanes& L,
                                         const StateT<D>& st) {
  FinishedT<D> f;
  finish(U, L, st, f);
  store_finished(p, f);
}

// LDS reads of a slot are inline asm: the compiler then neither orders them
// after every direct-to-LDS load in flight (its alias analysis cannot tell
// the slots apart, so it would wait for all of them) nor moves them; the
// waits are explicit (wait_vmcnt before, chunk_ready after).
__device__ __forceinline__ uint32_t lds_offset(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) char*)(p)));
}
template <int kOff>
__device__ __forceinline__ u32x4 ds_read16(uint32_t a) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(kOff));
  return v;
}
template <int kOff>
__device__ __forceinline__ u32x2 ds_read8(uint32_t a) {
  u32x2 v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(kOff));
  return v;
}
__device__ __forceinline__ float ds_read4(uint32_t a) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(a));
  return v;
}
// Waits for the slot reads and ties every register they wrote to the wait,
// so that no use is scheduled before it.
__device__ __forceinline__ void chunk_ready(Chunk& ch) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(ch.k[0][0]), "+v"(ch.k[0][1]), "+v"(ch.k[1][0]), "+v"(ch.k[1][1]),
                 "+v"(ch.v[0]), "+v"(ch.v[1]), "+v"(ch.v[2]), "+v"(ch.v[3]), "+v"(ch.v[4]),
                 "+v"(ch.v[5]), "+v"(ch.v[6]), "+v"(ch.v[7]), "+v"(ch.sc)
               :
               : "memory");
}

// Per-lane LDS offsets of the consumer's reads within a slot (lane (r, g):
// K of keys r and 16 + r at pieces 2g, 2g + 1; V of the 8 keys tv(e) at
// bytes 8r; one scale), independent of the chunk.
struct ReadOffsets {
  uint32_t k[2];  // + 2048 for keys 16..31
  uint32_t v[4];  // index e & 3; + 2048 for e >= 4
  uint32_t s;
};

__device__ __forceinline__ ReadOffsets read_offsets(int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  ReadOffsets o;
#pragma unroll
  for (int h = 0; h < 2; ++h) o.k[h] = kSlotK + swz(r16, 2 * g + h);
#pragma unroll
  for (int q = 0; q < 4; ++q) o.v[q] = kSlotV + swz(4 * g + q, r16 >> 1) + 8 * (r16 & 1);
  const int e = r16 & 7;
  const int key = 16 * (e >> 2) + 4 * g + (e & 3);
  o.s = kSlotScale + (r16 < 8 ? 0 : 128) + 4 * key;
  return o;
}

__device__ __forceinline__ void read_chunk(uint32_t base, const ReadOffsets& o, Chunk& ch) {
  const uint32_t k0 = base + o.k[0], k1 = base + o.k[1];
  ch.k[0][0] = ds_read16<0>(k0);
  ch.k[0][1] = ds_read16<0>(k1);
  ch.k[1][0] = ds_read16<2048>(k0);
  ch.k[1][1] = ds_read16<2048>(k1);
  const uint32_t v0 = base + o.v[0], v1 = base + o.v[1], v2 = base + o.v[2], v3 = base + o.v[3];
  ch.v[0] = ds_read8<0>(v0);
  ch.v[1] = ds_read8<0>(v1);
  ch.v[2] = ds_read8<0>(v2);
  ch.v[3] = ds_read8<0>(v3);
  ch.v[4] = ds_read8<2048>(v0);
  ch.v[5] = ds_read8<2048>(v1);
  ch.v[6] = ds_read8<2048>(v2);
  ch.v[7] = ds_read8<2048>(v3);
  ch.sc = ds_read4(base + o.s);
  chunk_ready(ch);
}

// Waits until at most `younger` vector memory operations are outstanding:
// with in-order completion, that is until everything issued before the last
// `younger` operations has completed. `younger` is wave-uniform; counts
// outside the listed ones fall back to a full wait.
__device__ __forceinline__ void wait_vmcnt_dyn(int younger) {
  switch (younger) {
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;
    case 10: wait_vmcnt<10>(); break;
    case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break;
    case 13: wait_vmcnt<13>(); break;
    case 14: wait_vmcnt<14>(); break;
    case 15: wait_vmcnt<15>(); break;
    case 16: wait_vmcnt<16>(); break;
    case 17: wait_vmcnt<17>(); break;
    case 18: wait_vmcnt<18>(); break;
    default: wait_vmcnt<0>(); break;
  }
}

}  // namespace
}  // namespace pa
