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

// Splits: the live count is within [1, num_splits] and [count/4 rounded up];
// the live ranges partition the tiles and differ by at most one.
static void splits() {
  for (int count = 0; count <= 600; ++count)
    for (int S = 1; S <= 300; S += (S < 20 ? 1 : 7)) {
      const int live = live_splits(count, S);
      CHECK(live >= 1 && live <= S, "live %d", live);
      CHECK(live == S || live == (count + kMinTilesPerSplit - 1) / kMinTilesPerSplit ||
                (count == 0 && live == 1),
            "live rule");
      int prev = 0, mn = 1 << 30, mx = -1;
      for (int s = 0; s < live; ++s) {
        int b, e;
        split_range(s, live, count, b, e);
        CHECK(b == prev && e >= b, "partition");
        prev = e;
        mn = e - b < mn ? e - b : mn;
        mx = e - b > mx ? e - b : mx;
      }
      CHECK(prev == count && mx - mn <= 1, "cover/balance");
      if (count >= live) CHECK(mn >= 1, "no empty live split when tiles suffice");
    }
  // request_splits is the live count of the request's widest row tile.
  for (int L = 1; L <= 5000; L += 37)
    for (int q : {1, 4, 16, 33})
      for (int W : {0, 100, 2048})
        for (int c = 0; c < 2; ++c) {
          if (q > L) continue;
          const int bq = 16;
          int want = 0;
          for (int j = 0; j < request_row_tiles(q, bq); ++j) {
            const RowTile t = request_tile(0, 0, q, L, bq, j);
            const int rb = W > 0 ? range_begin(t, W) : 0;
            const int n = kv_tile_count(rb, range_end(t, W, c));
            const int l = live_splits(n, 256);
            want = l > want ? l : want;
          }
          const int got = request_splits(q, L, bq, W, c, 256);
          // Without a window the last tile is the widest. With one, a full
          // tile before a short last tile can reach a few more keys; the
          // count then only changes the balance (a tile with fewer KV tiles
          // than live splits leaves some empty, which write lse = -inf).
          if (W == 0) CHECK(got == want, "request_splits L=%d q=%d W=%d", L, q, W);
          CHECK(got <= want, "request_splits above the widest tile's count");
          CHECK(got >= 1 && got <= 256, "range");
        }
  CHECK(request_splits(0, 10, 4, 0, true, 8) == 0, "empty request");
  std::printf("splits ok\n");
}

int main() {
  div32();
  row_tiles();
  visible();
  splits();
  std::printf("ALL OK\n");
  return fails;
}
