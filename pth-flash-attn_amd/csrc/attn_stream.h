// attn_stream.h -- device-side walk of the split partition (num_splits > 1),
// shared by the attention kernel (which computes the splits), the combine
// (which merges them) and the unused-split fill. The partition itself is
// defined in attn_geometry.h: the 32-key chunk streams of all (request, row
// tile, group of kGroupUnits KV-head units) laid end to end, work-group b of
// the attention grid taking positions [b per, (b + 1) per).
//
// Everything here is a pure function of query_start_loc, seq_lens and the
// launch constants, evaluated on the device, so a captured graph replays
// correctly as the lengths grow.

#pragma once

#include "attn_internal.h"

namespace pa {

// A kernel's launch parameters as values: the kernel argument is read at
// kernel entry by one vector load per lane (dword i of the argument segment
// in lane i % 64 of one of two registers: one memory round trip), and every
// field is taken from those registers by a lane read. Left to itself, the
// compiler reads the argument segment with scalar loads near each use and,
// under scalar-register pressure, reads fields again later: several
// dependent memory round trips on every wave's way to its first chunk.
template <class Params>
__device__ __forceinline__ Params params_in_registers(const Params& a, int lane) {
  static_assert(sizeof(Params) % 4 == 0, "dword-sized parameters");
  constexpr int kWords = static_cast<int>(sizeof(Params) / 4);
  static_assert(kWords <= 128, "parameters fit two registers of 64 lanes");
  const uint32_t* src = reinterpret_cast<const uint32_t*>(&a);
  uint32_t v0 = lane < kWords ? src[lane] : 0u;
  uint32_t v1 = lane + 64 < kWords ? src[lane + 64] : 0u;
  asm volatile("" : "+v"(v0), "+v"(v1));
  uint32_t w[kWords];
#pragma unroll
  for (int i = 0; i < kWords; ++i) w[i] = __builtin_amdgcn_readlane(i < 64 ? v0 : v1, i & 63);
  Params r;
  __builtin_memcpy(&r, w, sizeof(w));
  return r;
}

// Read-only inputs (query_start_loc, seq_lens, block_table) are read through
// the constant address space: a wave-uniform index then becomes a scalar
// load, which is tracked by lgkmcnt and never makes the wave wait for its
// vector loads in flight.
__device__ __forceinline__ int32_t ld_ro(const int32_t* base, int64_t i) {
  return ((const int32_t __attribute__((address_space(4)))*)(base))[i];
}

// What the layout depends on.
struct StreamDesc {
  const int32_t* qsl;
  const int32_t* seq_lens;
  int32_t num_reqs;
  int32_t bq;
  int32_t window;
  int32_t causal;
  int32_t n_hg;      // stream groups (of group_units(n_hu) KV-head units) per row tile
  int32_t num_wg;    // work-groups of the attention grid
  int32_t num_splits;
};

__device__ __forceinline__ int64_t readlane64(int64_t x, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(x), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32), l);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Wave-wide reductions by DPP lane moves (register to register, a few
// cycles each) instead of __shfl (ds_bpermute: an LDS crossbar round trip of
// ~100 cycles, and a chain of them sat on every work-group's start path).
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, kRowMask, 0xf, true);
}

// Inclusive prefix sum over the 64 lanes: within each row of 16 lanes by
// row shifts of 1, 2, 4 and 8 (lanes shifted in from outside the row add 0),
// then lane 15's running total into rows 1 and 3 and lane 31's into rows 2
// and 3 (row broadcasts).
__device__ __forceinline__ int32_t wave_scan32(int32_t x) {
  x += dpp_i32<0x111>(x);       // row_shr:1
  x += dpp_i32<0x112>(x);       // row_shr:2
  x += dpp_i32<0x114>(x);       // row_shr:4
  x += dpp_i32<0x118>(x);       // row_shr:8
  x += dpp_i32<0x142, 0xa>(x);  // row_bcast:15 (rows 1, 3)
  x += dpp_i32<0x143, 0xc>(x);  // row_bcast:31 (rows 2, 3)
  return x;
}

// Inclusive prefix sum over the 64 lanes. Values in [0, 2^24) (stream
// positions of one request, always in practice) take the 32-bit DPP scan;
// otherwise a 64-bit shift-up scan.
__device__ __forceinline__ int64_t wave_scan64(int64_t x, int lane) {
  if (__ballot(static_cast<uint64_t>(x) >= (1u << 24)) == 0)
    return wave_scan32(static_cast<int32_t>(x));
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t v = __shfl_up(x, d);
    if (lane >= d) x += v;
  }
  return x;
}

// Maximum over the 64 lanes (every lane): a butterfly within each row of 16
// lanes (quad swaps, half-row and row mirrors), then the four row maxima.
__device__ __forceinline__ int32_t wave_max32(int32_t x) {
  x = max(x, dpp_i32<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = max(x, dpp_i32<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = max(x, dpp_i32<0x141>(x));  // row_half_mirror
  x = max(x, dpp_i32<0x140>(x));  // row_mirror
  const int32_t a = max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16));
  const int32_t b = max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48));
  return max(a, b);
}

// Stream positions of request r (all its row tiles and groups) and the chunk
// count of its longest row tile.
__device__ __forceinline__ void request_positions(const StreamDesc& d, int r, int64_t& pos,
                                                  int32_t& longest) {
  int q0 = d.qsl[r], q1 = d.qsl[r + 1], sl = d.seq_lens[r];
  // All three loads in flight together: left to itself the compiler sinks
  // the seq_lens load into request_spans' tile loop, behind the wait for
  // the qsl loads, which made the partition two dependent round trips.
  asm volatile("" : "+v"(q0), "+v"(q1), "+v"(sl));
  int32_t sum, mx;
  request_spans(q1 - q0, sl, d.bq, d.window, d.causal != 0, sum, mx);
  pos = static_cast<int64_t>(sum) * d.n_hg;
  longest = mx;
}

// Total stream positions and the positions per work-group (every lane).
__device__ __forceinline__ int64_t stream_per(const StreamDesc& d, int lane, int64_t& total) {
  int64_t sum = 0;
  int32_t mx = 0;
  for (int r0 = 0; r0 < d.num_reqs; r0 += 64) {
    const int r = r0 + lane;
    if (r < d.num_reqs) {
      int64_t pos;
      int32_t longest;
      request_positions(d, r, pos, longest);
      sum += pos;
      mx = longest > mx ? longest : mx;
    }
  }
  total = readlane64(wave_scan64(sum, lane), 63);
  return chunks_per_group(total, wave_max32(mx), d.num_wg, d.num_splits);
}

// Stream positions of all requests before request r (every lane).
__device__ __forceinline__ int64_t positions_before(const StreamDesc& d, int r, int lane) {
  int64_t sum = 0;
  for (int r0 = 0; r0 < r; r0 += 64) {
    const int q = r0 + lane;
    if (q < r) {
      int64_t pos;
      int32_t longest;
      request_positions(d, q, pos, longest);
      sum += pos;
    }
  }
  return readlane64(wave_scan64(sum, lane), 63);
}

// One stream: row tile t, group hg, n chunks, positions [c0, c0 +
// stream_span(n)) (chunk c at position c0 + kStreamStartPositions + c); chunk
// c covers keys [cb + 32 c, cb + 32 c + 32).
struct StreamPos {
  RowTile t;
  int32_t hg;
  int64_t c0;
  int32_t n;
  int32_t cb;
};

// Forward-only cursor over the requests, 64 at a time, with each lane's
// inclusive prefix of stream positions.
struct StreamCursor {
  int r0 = -64;
  int64_t base = 0;  // positions before request r0
  int64_t end = 0;   // positions through request r0 + 63
  int64_t incl = 0;
};

// stream_per that also loads the cursor's first window when the launch has
// at most 64 requests: the loads that size the partition then also serve the
// first stream_locate, which otherwise reads the requests' lengths again
// before it can find the wave's first stream (one memory round trip fewer
// on the way to the first chunk).
__device__ __forceinline__ int64_t stream_per_cursor(const StreamDesc& d, int lane,
                                                     int64_t& total, StreamCursor& c) {
  if (d.num_reqs > 64) return stream_per(d, lane, total);
  int64_t pos = 0;
  int32_t mx = 0;
  if (lane < d.num_reqs) request_positions(d, lane, pos, mx);
  c.r0 = 0;
  c.base = 0;
  c.incl = wave_scan64(pos, lane);
  c.end = readlane64(c.incl, 63);
  total = c.end;
  return chunks_per_group(total, wave_max32(mx), d.num_wg, d.num_splits);
}

// The stream holding position P (P never decreases on a cursor). False when
// P is past the last stream.
__device__ __forceinline__ bool stream_locate(const StreamDesc& d, StreamCursor& c, int64_t P,
                                              int lane, StreamPos& out) {
  while (P >= c.end) {
    c.r0 += 64;
    if (c.r0 >= d.num_reqs) return false;
    c.base = c.end;
    const int r = c.r0 + lane;
    int64_t pos = 0;
    int32_t longest;
    if (r < d.num_reqs) request_positions(d, r, pos, longest);
    c.incl = wave_scan64(pos, lane);
    c.end = c.base + readlane64(c.incl, 63);
  }
  const int64_t local = P - c.base;
  const int j = static_cast<int>(__popcll(__ballot(c.incl <= local)));
  // r is wave-uniform; saying so makes the three reads scalar loads, and the
  // empty asm keeps them in flight together (otherwise the seq_lens read is
  // sunk into the tile loop below, behind the wait for the qsl reads).
  const int r = __builtin_amdgcn_readfirstlane(c.r0 + j);
  int64_t at = c.base + (j > 0 ? readlane64(c.incl, j - 1) : 0);
  int q_start = ld_ro(d.qsl, r), q_end = ld_ro(d.qsl, r + 1), seq_len = ld_ro(d.seq_lens, r);
  asm volatile("" : "+s"(q_start), "+s"(q_end), "+s"(seq_len));
  const int q_len = q_end - q_start;
  const int tiles = request_row_tiles(q_len, d.bq);
  for (int k = 0; k < tiles; ++k) {
    const RowTile t = request_tile(r, q_start, q_len, seq_len, d.bq, k);
    const int32_t n = tile_chunks(t, d.window, d.causal != 0);
    const int32_t sn = stream_span(n);
    const int64_t span = static_cast<int64_t>(sn) * d.n_hg;
    if (P < at + span) {
      out.t = t;
      out.hg = static_cast<int32_t>((P - at) / sn);
      out.n = n;
      out.c0 = at + static_cast<int64_t>(out.hg) * sn;
      out.cb = tile_chunk_base(t, d.window);
      return true;
    }
    at += span;
  }
  return false;  // not reached: P < c.end lies in some tile of request r
}

}  // namespace pa
