// Host checks of attn_geometry.h, built with g++ by tests/test_geometry.py.
// Each check is against a brute-force restatement on small domains (the
// reference tests the same header family this way: tests/cpp/test_geometry.cpp
// of the reference checks its FastDivmod premises and stride arithmetic).
// Prints one line per check and exits non-zero on the first failure.

#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "attn_geometry.h"

using namespace pa;

static int fails = 0;
#define CHECK(cond, ...)                                       \
  do {                                                         \
    if (!(cond)) {                                             \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                       \
      std::fprintf(stderr, "\n");                              \
      std::exit(1);                                            \
    }                                                          \
  } while (0)

// n / d for every n < 2^16 and d <= 512, and for n near the top of the
// domain, near multiples of d and at random, for d up to 2^31 - 1.
static void div32() {
  for (uint32_t d = 1; d <= 512; ++d) {
    const Div32 v = Div32::make(d);
    for (uint32_t n = 0; n < (1u << 16); ++n) CHECK(v.div(n) == n / d, "n=%u d=%u", n, d);
  }
  std::mt19937_64 rng(1);
  const uint32_t top = 0x7fffffffu;
  std::vector<uint32_t> ds = {1, 2, 3, 5, 7, 16, 17, 64, 528, 816, 1000003, 1u << 20,
                              (1u << 30) + 1, top - 1, top};
  for (int i = 0; i < 2000; ++i) ds.push_back(1 + static_cast<uint32_t>(rng() % top));
  for (uint32_t d : ds) {
    const Div32 v = Div32::make(d);
    auto chk = [&](uint64_t n) {
      if (n > top) return;
      CHECK(v.div(static_cast<uint32_t>(n)) == n / d, "n=%llu d=%u", (unsigned long long)n, d);
    };
    for (uint64_t n = top - 64; n <= top; ++n) chk(n);
    for (uint64_t k = 1; k < 64 && k * d <= top + uint64_t{1}; ++k) {
      chk(k * d - 1);
      chk(k * d);
      chk(k * d + 1);
    }
    for (int i = 0; i < 2000; ++i) chk(rng() % (uint64_t{top} + 1));
  }
  std::printf("div32 ok\n");
}

// Row tiles: the tiles of each request cover its tokens exactly once, every
// index below T / bq + R is either a tile of some request or empty, and the
// request search agrees with a linear scan.
static void row_tiles() {
  std::mt19937 rng(2);
  for (int trial = 0; trial < 3000; ++trial) {
    const int R = 1 + rng() % 20;
    const int bq = 1 + rng() % 64;
    std::vector<int32_t> qsl(R + 1, 0), sl(R);
    for (int r = 0; r < R; ++r) {
      const int q = (rng() % 4 == 0) ? 0 : 1 + rng() % 100;
      qsl[r + 1] = qsl[r] + q;
      sl[r] = q + rng() % 300;
    }
    const int T = qsl[R];
    const Div32 bd = Div32::make(bq);
    const int upper = T / bq + R;
    std::vector<int> seen(T, 0);
    for (int x = 0; x < upper + 3; ++x) {
      RowTile t;
      if (!row_tile(qsl.data(), sl.data(), bd, R, x, t)) continue;
      CHECK(x < upper, "tile %d beyond q_tiles_upper %d", x, upper);
      int lin = 0;
      while (lin + 1 < R && (qsl[lin + 1] / bq + lin + 1) <= x) ++lin;
      CHECK(t.req == lin, "request of tile %d: %d vs %d", x, t.req, lin);
      CHECK(t.num_tok >= 1 && t.num_tok <= bq, "num_tok %d", t.num_tok);
      for (int i = 0; i < t.num_tok; ++i) ++seen[t.q_start + t.tok_begin + i];
      // request_tile reproduces row_tile for the same tile of the request.
      const RowTile u = request_tile(t.req, t.q_start, t.q_len, t.seq_len, bq, t.tok_begin / bq);
      CHECK(u.tok_begin == t.tok_begin && u.num_tok == t.num_tok, "request_tile");
    }
    for (int i = 0; i < T; ++i) CHECK(seen[i] == 1, "token %d covered %d times", i, seen[i]);
    for (int r = 0; r < R; ++r)
      CHECK(request_row_tiles(qsl[r + 1] - qsl[r], bq) == (qsl[r + 1] - qsl[r] + bq - 1) / bq,
            "row tiles");
  }
  std::printf("row_tiles ok\n");
}

// Visible ranges against the mask definition (vLLM's, restated by the
// reference at python/pth_testing/reference.py:553-572): causal k <= p,
// non-causal k < L, and with a window |p - k| < W.
static void visible() {
  for (int L = 1; L <= 70; ++L)
    for (int q = 1; q <= L && q <= 9; ++q)
      for (int W : {0, 1, 2, 3, 5, 16, 64, 100})
        for (int causal = 0; causal < 2; ++causal) {
          const RowTile t = request_tile(0, 0, q, L, q, 0);
          for (int tok = 0; tok < q; ++tok) {
            const int p = L - q + tok;
            int lo = -1, hi = -2;
            for (int k = 0; k < L; ++k) {
              bool ok = causal ? k <= p : true;
              if (W > 0) ok = ok && std::abs(p - k) < W;
              if (ok) {
                if (lo < 0) lo = k;
                hi = k;
              }
            }
            CHECK(key_lo(t, tok, W) == lo && key_hi(t, tok, W, causal) == hi,
                  "L=%d q=%d W=%d causal=%d tok=%d: [%d,%d] vs [%d,%d]", L, q, W, causal, tok,
                  key_lo(t, tok, W), key_hi(t, tok, W, causal), lo, hi);
            // The tile range contains every token's range.
            CHECK(range_begin(t, W) <= lo && range_end(t, W, causal) > hi, "tile range");
          }
        }
  std::printf("visible ok\n");
}

// The chunk streams of the split partition: a row tile's chunks cover every
// key its rows see, and no chunk is wholly outside them; the per-work-group
// share keeps every stream within num_splits work-groups; stream_splits
// names exactly the work-groups whose ranges meet the stream.
static void streams() {
  for (int L = 1; L <= 300; L += 7)
    for (int q = 1; q <= L && q <= 40; q += 3)
      for (int W : {0, 1, 5, 33, 64, 100})
        for (int causal = 0; causal < 2; ++causal)
          for (int bq : {1, 4, 16}) {
            int32_t sum = 0, mx = 0;
            request_spans(q, L, bq, W, causal, sum, mx);
            int32_t s2 = 0, m2 = 0;
            for (int j = 0; j < request_row_tiles(q, bq); ++j) {
              const RowTile t = request_tile(0, 0, q, L, bq, j);
              const int cb = tile_chunk_base(t, W);
              const int n = tile_chunks(t, W, causal);
              CHECK(cb % kChunkTokens == 0 && n >= 1, "chunk base / count");
              bool first_used = false, last_used = false;
              for (int tok = t.tok_begin; tok < t.tok_begin + t.num_tok; ++tok) {
                const int lo = key_lo(t, tok, W), hi = key_hi(t, tok, W, causal);
                CHECK(lo >= cb && hi < cb + kChunkTokens * n, "chunks cover the keys");
                first_used |= lo < cb + kChunkTokens;
                last_used |= hi >= cb + kChunkTokens * (n - 1);
              }
              CHECK(first_used && last_used, "no chunk wholly outside the keys");
              s2 += n + kStreamStartPositions;
              m2 = n > m2 ? n : m2;
            }
            CHECK(sum == s2 && mx == m2, "request_spans");
          }
  std::mt19937 rng(3);
  for (int trial = 0; trial < 4000; ++trial) {
    const int nstreams = 1 + rng() % 40;
    std::vector<int> len(nstreams);
    int64_t total = 0;
    int32_t mx = 0;
    for (int& n : len) {
      n = 1 + rng() % (trial % 3 == 0 ? 5000 : 200);
      total += stream_span(n);
      mx = n > mx ? n : mx;
    }
    const int num_wg = 1 + rng() % 300;
    const int S = 2 + rng() % 300;
    const int64_t per = chunks_per_group(total, mx, num_wg, S);
    CHECK(per >= kMinChunksPerSplit && per * num_wg + kStreamStartPositions >= total,
          "per covers the total");
    // Per work-group: its chunks plus kStreamStartPositions per unit (a
    // stream whose chunks its range meets) never exceed per plus one start.
    std::vector<int64_t> cost(num_wg, 0);
    int64_t c0 = 0;
    for (int n : len) {
      int first, live;
      stream_splits(c0, n, per, first, live);
      CHECK(live >= 1 && live <= S, "live %d > S %d (n=%d per=%lld)", live, S, n, (long long)per);
      // Brute force: the work-groups whose range meets the chunk positions
      // [c0 + start, c0 + start + n).
      const int64_t cs = c0 + kStreamStartPositions;
      int bf_first = -1, bf_count = 0;
      for (int b = 0; b < num_wg; ++b) {
        const int64_t lo = b * per + kStreamStartPositions, hi = lo + per;
        if (lo < cs + n && hi > cs) {
          if (bf_first < 0) bf_first = b;
          ++bf_count;
          const int64_t a = lo > cs ? lo : cs, e = hi < cs + n ? hi : cs + n;
          cost[b] += (e - a) + kStreamStartPositions;
        }
      }
      CHECK(bf_first == first && bf_count == live, "stream_splits");
      c0 += stream_span(n);
    }
    for (int b = 0; b < num_wg; ++b)
      CHECK(cost[b] <= per + kStreamStartPositions, "work-group %d cost %lld > per %lld + start", b,
            (long long)cost[b], (long long)per);
  }
  std::printf("streams ok\n");
}

// cell_reach_fits: a layout whose furthest byte is within one row of 4 GiB
// must be refused for D = 256 rows even when it fits for shorter rows (the
// 32-bit offsets of the cell kernels would wrap), and the vLLM cell must fit.
static void cell_reach() {
  const uint64_t lim = uint64_t{1} << 32;
  // vLLM NHD cell, 8 heads, D = 128: tiny reach.
  CHECK(cell_reach_fits(2112, 264, 8, 260, 128), "vLLM cell");
  // Brute force over head sizes and the last bytes below 4 GiB.
  const int32_t ds[3] = {64, 128, 256};
  for (int32_t d : ds) {
    for (uint64_t gap = 0; gap < 600; ++gap) {
      // 15 slot strides + 7 head strides + max offset = lim - gap.
      const uint64_t ss = 200000000, sh = 1000;
      const uint64_t base = 15 * ss + 7 * sh;
      const uint64_t max_off = lim - gap - base;
      const bool want = gap > static_cast<uint64_t>(d);  // last byte read: max_off + d - 1 < lim
      CHECK(cell_reach_fits(ss, sh, 8, max_off, d) == want, "d=%d gap=%llu", d,
            static_cast<unsigned long long>(gap));
    }
  }
  // A reach that fits a 128-byte row but not a 256-byte one.
  const uint64_t ss = 1u << 20, sh = 264;
  const uint64_t max_off = lim - 15 * ss - 7 * sh - 200;
  CHECK(cell_reach_fits(ss, sh, 8, max_off, 128), "128-byte rows fit");
  CHECK(!cell_reach_fits(ss, sh, 8, max_off, 256), "256-byte rows must not fit");
  std::printf("cell_reach ok\n");
}

int main() {
  div32();
  row_tiles();
  visible();
  streams();
  cell_reach();
  std::printf("ALL OK\n");
  return fails;
}
