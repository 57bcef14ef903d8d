// attn_geometry.h -- integer geometry of one attention launch, shared by the
// gfx950 kernels and the host launcher (and compiled by g++ for the CPU
// tests by tests/cpp/test_geometry.cpp).
//
// It answers, with integer arithmetic only:
//   * division by run-time divisors (block size, GQA group, row-tile height)
//     as one multiply-high and a shift;
//   * which request and query tokens a row tile x owns (the q-tile numbering
//     of vLLM's unified attention, reference cache_geometry.cuh:336-394);
//   * the visible key range [lo, hi] of a query token (causal, sliding
//     window, non-causal; reference cache_geometry.cuh:396-468);
//   * how the keys of all row tiles are cut into splits: an even share of
//     32-key chunks per work-group (the reference cuts each row tile's KV
//     tiles into num_splits near-equal ranges, cache_geometry.cuh:426-432,
//     506-515; here the cut is global, so no work-group idles and short
//     requests are not split at all).
// Header-only; needs <stdint.h> only.

#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define PA_HD __host__ __device__ __forceinline__
#else
#define PA_HD inline
#endif

namespace pa {

// KV tokens per tile of the reference's split partition (the planner's
// KV_TILE_TOKENS; reference tile_traits.cuh / planner.py:98): the unit its
// window cap on num_splits counts in, reported by pth_attn_tiling.
constexpr int32_t kTileTokens = 64;
// KV tokens per softmax step of one wave (two 16-token MFMA column blocks).
constexpr int32_t kChunkTokens = 32;
// Query rows per wave: the N of a 16x16x32 MFMA.
constexpr int32_t kRowsPerWave = 16;
// Waves per work-group of the combine kernel.
constexpr int32_t kWaves = 4;
// Waves per work-group of the attention kernel: the KV-head units of one
// stream group, one per wave.
constexpr int32_t kGroupUnits = 8;

// KV-head units per stream group: the row tile's units rounded up to a power
// of two, at most kGroupUnits. A work-group of kGroupUnits waves holds
// kGroupUnits / group_units(n_hu) groups' worth of waves, and the split
// partition counts that many partition work-groups per work-group, so a row
// tile with fewer units than waves (few KV heads, a single row group) still
// keeps every wave of the work-group streaming.
// Whether every byte the cell-view kernels address from one page stays
// within 32-bit offsets of the page's base: a 16-key group (15 slot strides),
// any KV head, any stream offset, plus the row the kernel reads there (one
// head_size-byte K or V row; the scale streams need 4 of those bytes).
// The cell-view kernels form uint32 offsets, so a layout that reaches 4 GiB
// must take the 64-bit-address kernels.
PA_HD bool cell_reach_fits(uint64_t slot_stride, uint64_t head_stride, int32_t num_kv_heads,
                           uint64_t max_stream_off, int32_t head_size) {
  const uint64_t lim = uint64_t{1} << 32;
  const uint64_t reach = 15u * slot_stride +
                         static_cast<uint64_t>(num_kv_heads - 1) * head_stride +
                         max_stream_off + static_cast<uint64_t>(head_size);
  return reach < lim;
}

PA_HD int32_t group_units(int32_t n_hu) {
  int32_t g = 1;
  while (g < n_hu && g < kGroupUnits) g <<= 1;
  return g;
}

PA_HD uint32_t mulhi32(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umulhi(a, b);
#else
  return static_cast<uint32_t>((static_cast<uint64_t>(a) * b) >> 32);
#endif
}

// Exact n / d for 0 <= n < 2^31 and 1 <= d < 2^31.
// Construction: s = ceil(log2 d), p = 31 + s, m = ceil(2^p / d) (< 2^32).
// With m d = 2^p + e, 0 <= e < d <= 2^s, n m / 2^p = n / d + n e / (d 2^p)
// and n e < 2^31 2^s = 2^p, so the error term is below 1/d and the floor
// is exact (Granlund & Montgomery, PLDI 1994, Thm 4.2). d = 1 is the
// identity (mul = 0 marks it).
struct Div32 {
  uint32_t d;
  uint32_t mul;
  uint32_t shift;  // p - 32 = s - 1

  static Div32 make(uint32_t dv) {
    Div32 r{dv, 0u, 0u};
    if (dv <= 1u) return r;
    uint32_t s = 0;
    while ((uint64_t{1} << s) < dv) ++s;
    const uint64_t two_p = uint64_t{1} << (31 + s);
    r.mul = static_cast<uint32_t>((two_p + dv - 1) / dv);
    r.shift = s - 1;
    return r;
  }
  PA_HD uint32_t div(uint32_t n) const {
    return mul == 0u ? n : (mulhi32(n, mul) >> shift);
  }
};

// One row tile of query tokens of one request.
struct RowTile {
  int32_t req;        // request index
  int32_t tok_begin;  // first query token of the tile within the request
  int32_t num_tok;    // query tokens in the tile (1..bq)
  int32_t q_len;      // query tokens of the request
  int32_t seq_len;    // KV length of the request, new tokens included
  int32_t q_start;    // global index of the request's first query token
};

// Request r owns the tile indices [qsl[r] / bq + r, qsl[r+1] / bq + r + 1):
// at least ceil(q_len / bq) tiles, and the last request ends at or below
// T / bq + R, the planner's q_tiles_upper (reference cache_geometry.cuh:336-350).
PA_HD int32_t first_tile_of(const int32_t* qsl, const Div32& bq, int32_t r) {
  return static_cast<int32_t>(bq.div(static_cast<uint32_t>(qsl[r]))) + r;
}

// Largest r in [0, R) with first_tile_of(r) <= x (strictly increasing in r).
PA_HD int32_t request_of_tile(const int32_t* qsl, const Div32& bq, int32_t R,
                              int32_t x) {
  int32_t lo = 0, hi = R - 1;
  while (lo < hi) {
    const int32_t mid = (lo + hi + 1) >> 1;
    if (first_tile_of(qsl, bq, mid) <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Fills t for row tile x; false when the tile holds no query token.
PA_HD bool row_tile(const int32_t* qsl, const int32_t* seq_lens,
                    const Div32& bq, int32_t R, int32_t x, RowTile& t) {
  if (R <= 0) return false;
  const int32_t r = request_of_tile(qsl, bq, R, x);
  t.req = r;
  t.q_start = qsl[r];
  t.q_len = qsl[r + 1] - t.q_start;
  t.seq_len = seq_lens[r];
  const int64_t begin =
      static_cast<int64_t>(x - first_tile_of(qsl, bq, r)) * static_cast<int64_t>(bq.d);
  if (begin >= t.q_len) return false;
  t.tok_begin = static_cast<int32_t>(begin);
  const int32_t left = t.q_len - t.tok_begin;
  t.num_tok = left < static_cast<int32_t>(bq.d) ? left : static_cast<int32_t>(bq.d);
  return true;
}

// Absolute KV position of query token `tok` of the request (bottom-right).
PA_HD int32_t query_pos(const RowTile& t, int32_t tok) {
  return t.seq_len - t.q_len + tok;
}

// Inclusive visible key range of query token `tok` (reference
// reference.py:553-593 visible_mask / visible_bounds).
PA_HD int32_t key_lo(const RowTile& t, int32_t tok, int32_t window) {
  const int32_t p = query_pos(t, tok);
  return (window > 0 && p >= window) ? p - window + 1 : 0;
}
PA_HD int32_t key_hi(const RowTile& t, int32_t tok, int32_t window,
                     bool causal) {
  const int32_t p = query_pos(t, tok);
  if (causal) return p;
  return (window > 0 && t.seq_len - 1 - p >= window) ? p + window - 1
                                                     : t.seq_len - 1;
}

// The keys any token of the tile sees: [range_begin, range_end). Both bounds
// are non-decreasing in the token, so they come from the first and the last
// token of the tile.
PA_HD int32_t range_begin(const RowTile& t, int32_t window) {
  return key_lo(t, t.tok_begin, window);
}
PA_HD int32_t range_end(const RowTile& t, int32_t window, bool causal) {
  return key_hi(t, t.tok_begin + t.num_tok - 1, window, causal) + 1;
}

// Row tile j (0-based) of a request: query tokens [j bq, min((j + 1) bq, q_len)).
PA_HD RowTile request_tile(int32_t req, int32_t q_start, int32_t q_len,
                           int32_t seq_len, int32_t bq, int32_t j) {
  RowTile t;
  t.req = req;
  t.q_start = q_start;
  t.q_len = q_len;
  t.seq_len = seq_len;
  t.tok_begin = j * bq;
  const int32_t left = q_len - t.tok_begin;
  t.num_tok = left < bq ? left : bq;
  return t;
}

// Row tiles of a request: ceil(q_len / bq).
PA_HD int32_t request_row_tiles(int32_t q_len, int32_t bq) {
  return (q_len + bq - 1) / bq;
}

// ---------------------------------------------------------------------------
// Split partition (num_splits > 1). The keys of every row tile, from a
// 32-aligned base, are a stream of 32-key chunks; the streams of all
// (request, row tile, group of 8 KV-head units) are laid end to end, in that
// order, each preceded by kStreamStartPositions positions that hold no chunk,
// and work-group b of the grid takes positions [b per + kStreamStartPositions,
// (b + 1) per + kStreamStartPositions) (the first stream's start positions
// are every work-group's own first start, so no range holds them). A stream
// cut by such a boundary is computed in parts (its splits), one per
// work-group whose range meets its chunks, and merged by the LSE combine.
// The start positions price what a wave pays to begin a unit (its
// block-table entry, query and first chunk arrive before its first chunk
// step): a work-group whose range runs into a new stream gets that many
// fewer chunks, so every work-group costs about per + one start, instead
// of those crossing a stream boundary costing a start more than the rest.
// A stream only has as many splits as the work-groups its chunks need.

// Positions in front of each stream's chunks. Per-wave timestamps put a
// unit's first chunk two to three chunk steps after the unit is known;
// measured over 1 to 4 (A/B in one process): config 4 -2.5 us with any of
// them, config 2 -1.5 / -2.8 / -3.3 / -1.4 us, so 3.
constexpr int32_t kStreamStartPositions = 3;

// Positions of a stream of n chunks.
PA_HD int32_t stream_span(int32_t n) { return n > 0 ? n + kStreamStartPositions : 0; }

// First key of chunk 0 of a row tile, and the number of chunks that cover the
// keys any of its rows sees.
PA_HD int32_t tile_chunk_base(const RowTile& t, int32_t window) {
  const int32_t rb = window > 0 ? range_begin(t, window) : 0;
  return rb & ~(kChunkTokens - 1);
}
PA_HD int32_t tile_chunks(const RowTile& t, int32_t window, bool causal) {
  const int32_t base = tile_chunk_base(t, window);
  const int32_t re = range_end(t, window, causal);
  return re > base ? (re - base + kChunkTokens - 1) / kChunkTokens : 0;
}

// Positions (the sum of stream_span) and the largest tile_chunks over the
// row tiles of a request.
PA_HD void request_spans(int32_t q_len, int32_t seq_len, int32_t bq, int32_t window,
                         bool causal, int32_t& sum, int32_t& max) {
  sum = 0;
  max = 0;
  const int32_t tiles = request_row_tiles(q_len, bq);
  for (int32_t j = 0; j < tiles; ++j) {
    const int32_t n = tile_chunks(request_tile(0, 0, q_len, seq_len, bq, j), window, causal);
    sum += stream_span(n);
    max = n > max ? n : max;
  }
}

// Stream positions per work-group: an even share of the `total` positions
// (less the first stream's start positions, which no range holds),
// but at least kMinChunksPerSplit and enough that no stream of up to `max_n`
// chunks meets more than num_splits work-groups (n consecutive chunk
// positions meet at most ceil((n - 1) / per) + 1 of them). One chunk is the floor: a small launch
// is a chain of dependent chunk loads per wave, so the shortest chain wins
// (measured: config 1's layer call 20.3 us with a floor of 4 chunks, 16.5 us
// with 1; long launches have shares far above the floor).
constexpr int32_t kMinChunksPerSplit = 1;
PA_HD int64_t chunks_per_group(int64_t total, int32_t max_n, int32_t num_wg, int32_t num_splits) {
  const int64_t ranged = total > kStreamStartPositions ? total - kStreamStartPositions : 0;
  int64_t per = (ranged + num_wg - 1) / num_wg;
  if (per < kMinChunksPerSplit) per = kMinChunksPerSplit;
  if (num_splits > 1 && max_n > 1) {
    const int64_t need = (static_cast<int64_t>(max_n) - 1 + num_splits - 2) / (num_splits - 1);
    if (per < need) per = need;
  }
  return per;
}

// The work-groups whose ranges meet the chunks of the stream of n chunks
// that starts at position c0: first and count (its splits); split s of the
// stream is work-group first + s. (Its chunks lie at [c0 + start, c0 + start
// + n) and range b starts at b per + start, so the start cancels.)
PA_HD void stream_splits(int64_t c0, int32_t n, int64_t per, int32_t& first, int32_t& live) {
  first = static_cast<int32_t>(c0 / per);
  live = n > 0 ? static_cast<int32_t>((c0 + n - 1) / per) - first + 1 : 1;
}

}  // namespace pa
