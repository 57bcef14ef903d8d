// attn_rows.hip -- the gfx950 row-block kernel: num_splits == 1 launches
// whose row tiles hold many query rows (chunked prefill, long verify
// windows, mixed prefill + decode batches), D = 128, paged cell caches.
//
// Why a second kernel. The unit kernels of attn_fwd.hip give every 16-row
// group its own wave and its own pass over the keys: right for decode, where
// the rows of a KV head are few and the bytes are read once, but a 2048-token
// prefill chunk has 8192 rows per KV head, and 512 passes over the same keys
// make the launch L2-bandwidth bound (and spend the int8 -> bf16 conversion
// 512 times per key). Here a work-group of 8 waves takes a *row block*: up to
// 256 rows (256 / G query tokens) of one request and one KV head, and the 8
// waves share one stream of 32-key chunks staged in LDS by direct-to-LDS
// loads, each wave computing its 32 rows (two 16-row MFMA groups that share
// the converted K and V operands) against every chunk.
//
// A row block with fewer rows (a decode token: G rows) has fewer row sets
// of 32 rows than waves; its waves then split the keys instead: RS row sets
// (RS a power of two) times KP = 8 / RS key parts, the parts' partial
// (O, m, l) merged through LDS at the end in a fixed order. So a long decode
// row in a mixed batch runs on 8 waves, not one, and no wave idles.
//
// Pipeline. Each part has a ring of 16 / KP chunk slots in LDS. At step k
// every wave waits for its own share of the loads of chunk k (the 9 loads of
// a chunk are spread over the RS waves of the part), then the work-group
// meets at a barrier, after which chunk k is complete in LDS and every wave
// has finished reading chunk k - 1, so chunk k + A (A chunks ahead) is
// issued into the slot that chunk k - 1 left, and chunk k is computed. The
// numerics are those of attn_fwd.hip's chunk step (reference
// attn_kernel.cuh:540-600, softmax.cuh:91-170).
//
// Work order. Blocks are (request, token block, KV head), KV head fastest,
// the requests of each group of 64 in decreasing order of estimated work, the
// token blocks of a request from its last (longest key range) to its first,
// dealt in rounds of W blocks (snake order, so long and short blocks pair
// up; the KV heads of a token block to work-groups on one XCD); each
// work-group walks its rounds from a rotated start (see BlockWalk).

#include "attn_device.h"

namespace pa {
namespace {

// PV operands of the row-block kernel are fp16: V as int8 -> fp16 (exact)
// and P'' = fp16(p vs 2^-C), the reference's precision class (reference
// softmax.cuh:91-170: fp16 P with the V scale folded in and a running
// V-scale exponent). C is the wave's running exponent of the largest V scale
// seen (every chunk's V scales < 2^C), so p vs 2^-C < 2^8 (p <= 2^8 under the
// lazy rescale) and fits fp16; when a chunk raises C, O is rescaled by
// 2^(C_old - C_new). fp16 keeps 11 significant bits against bf16's 8, so one
// PV product per operand suffices (the decode kernels, bandwidth-bound, keep
// their bf16 hi + lo pair).
__device__ __forceinline__ f32x4 mfma_f16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// Byte j of each of eight 8-byte runs -> eight fp16 (exact for int8).
__device__ __forceinline__ f16x8 column_to_f16(const u32x2 (&v)[8], int j) {
  const int w = j >> 2, b = j & 3;
  f16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = static_cast<_Float16>(i8_to_f32(v[e][w], b));
  return r;
}
// The running V-scale exponent before any chunk: no scale seen yet.
constexpr int kNoExp = -1000;
// The exponent e of a largest V scale v (v < 2^e), clamped to [-125, 126]
// (2^-e a normal float); kNoExp for v = 0 (every key masked). Wave-uniform.
__device__ __forceinline__ int vscale_exp(float v) {
  int e = v > 0.0f ? static_cast<int>((__builtin_bit_cast(uint32_t, v) >> 23) & 0xff) - 126
                   : kNoExp;
  e = e == kNoExp ? e : (e < -125 ? -125 : (e > 126 ? 126 : e));
  return __builtin_amdgcn_readfirstlane(e);
}
// After a wave's last chunk: O is in units of 2^-C, so O / (l 2^-C) is the
// output and m + C + log2(l 2^-C) = m + log2(l) the row's log2-sum-exp, the
// form finish() and the key-part merge expect.
__device__ __forceinline__ void undo_vexp(State& st, int vexp) {
  if (vexp == kNoExp) return;
  st.l *= __builtin_ldexpf(1.0f, -vexp);
  st.m += static_cast<float>(vexp);
}

constexpr int kRowWaves = kFwdWaves;              // waves per work-group
constexpr int kWaveRows = 2 * kRowsPerWave;       // rows per wave
constexpr int kBlockRows = kRowWaves * kWaveRows;  // rows per block
constexpr int kRowSlots = 16;                     // LDS chunk slots per work-group
constexpr int kRowAhead = 3;                      // chunks in flight per part, at most
// Partial state of one wave for the merge of key parts: O (2 groups x 8
// f32x4 per lane), then m and l (2 groups x 1 float per lane each).
constexpr int kMergeO = 2 * 8 * 16 * 64;
constexpr int kMergeBytes = kMergeO + 2 * 2 * 4 * 64;
static_assert((kRowWaves - 1) * kMergeBytes <= kRowSlots * kSlotBytes,
              "the merge area must fit the chunk slots");

__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// One row block, uniform across the work-group.
struct Block {
  RowTile t;
  int kvh;
  int rows;          // num_tok * G
  int log_rs;        // row sets of kWaveRows rows: RS = 1 << log_rs
  int kp;            // key parts: kRowWaves / RS
  int c_begin;       // first chunk's key (32-aligned)
  int n_chunks;      // chunks covering the keys of any row of the block
  int ld_lo, ld_hi;  // keys the block reads
};

template <bool kWindow>
__device__ __forceinline__ void make_block(const AttnParams& p, const RowTile& t, int kvh,
                                           Block& B) {
  const int window = kWindow ? p.window : 0;
  const bool causal = kWindow ? (p.causal != 0) : true;
  B.t = t;
  B.kvh = kvh;
  B.rows = t.num_tok * p.group;
  const int sets = (B.rows + kWaveRows - 1) / kWaveRows;
  int lr = 0;
  while ((1 << lr) < sets) ++lr;
  B.log_rs = lr;
  B.kp = kRowWaves >> lr;
  B.ld_lo = range_begin(t, window);
  B.ld_hi = range_end(t, window, causal);
  B.c_begin = B.ld_lo & ~(kChunkTokens - 1);
  B.n_chunks = B.c_begin < B.ld_hi ? (B.ld_hi - B.c_begin + kChunkTokens - 1) / kChunkTokens : 0;
}

// The blocks of one work-group, in order (a prefix sum over requests, 64 per
// wave instruction, as the unit table of attn_fwd.hip). Within each group of
// 64 requests the requests are taken in decreasing order of their estimated
// work (row tiles x keys per row), so that the snake of rounds (work-group b
// takes unit b of even rounds and W - 1 - b of odd ones) pairs long blocks
// with short ones and evens out the work-groups' totals (a mixed prefill +
// decode batch whose long decodes came last left some work-groups a decode
// block behind the others).
//
// Placement. Work-groups are dealt to the 8 XCDs in turn (work-group b on
// XCD b mod 8), and each XCD has its own L2. In a round of decode blocks,
// slot H t + h (KV head h of the round's t-th row tile) goes to work-group
// h M + t (M = W / H): the H heads of a row tile, whose 264-byte cells share
// 128-byte lines, run on one XCD. In a round of wide (prefill) blocks, slot
// s goes to work-group s: with H dividing 8, KV head h runs on the XCDs
// x with x mod H = h, so the row tiles of one head, which read the same keys, share
// an L2 (config 5: 4,562 -> 4,417 us; its prefill blocks had fetched 2.65 GB
// for their 0.2 GB of keys with one row tile's heads per XCD). A round is
// wide when its first unit lies among the wide requests' units, which rank
// first.
//
// Each work-group walks its rounds starting at round x mod R (R rounds in
// all, x its XCD) and wraps around: the same blocks, in a rotated order, all
// work-groups of an XCD in the same round (so the row tiles of a head or the
// heads of a row tile run at the same time). In a mixed batch the decode
// blocks (HBM-bound, ranked last) then run at different times on different
// XCDs, beside other XCDs' prefill blocks (MFMA-bound), instead of all at the
// end, where every unit streamed decode keys at once and HBM bounded them
// (config 5: 4.84 ms, the sum of its prefill part alone, 3.95 ms, and its
// decode part alone, 0.89 ms).
template <bool kWindow>
struct BlockWalk {
  int r0 = -64;
  int u0 = 0, u1 = 0;
  int incl = 0;
  int sreq = 0;  // lane k: the request (within the group) of rank k
  int round = 0;
  int total = -1;  // units of the launch (-1: not counted yet)
  int nrounds = 0;
  int rot = 0;     // the work-group's first round
  int n_wide = 0;  // units of wide-block requests (ranked first), first group only

  // Moves to the next group of 64 requests: their ranks and the prefix sum
  // of their units. False past the last request.
  __device__ __forceinline__ bool scan_group(const AttnParams& p, int lane) {
    r0 += 64;
    u0 = u1;
    if (r0 >= p.num_reqs) return false;
    const int r = r0 + lane;
    int tiles = 0;
    float work = -1.0f;  // lanes past the last request sort last
    if (r < p.num_reqs) {
      const int q_len = p.qsl[r + 1] - p.qsl[r];
      tiles = request_row_tiles(q_len, p.blk_tok);
      work = static_cast<float>(tiles) * static_cast<float>(p.seq_lens[r] - q_len / 2);
    }
    // Rank: requests with more work first, ties in request order.
    int rank = 0;
    for (int j = 0; j < 64; ++j) {
      const float wj =
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, work), j));
      rank += (wj > work || (wj == work && j < lane)) ? 1 : 0;
    }
    sreq = __builtin_amdgcn_ds_permute(rank * 4, lane);
    const int units = __builtin_amdgcn_ds_permute(rank * 4, tiles * p.num_kv_heads);
    int x = units;
#pragma unroll
    for (int dd = 1; dd < 64; dd <<= 1) {
      const int v = __shfl_up(x, dd);
      if (lane >= dd) x += v;
    }
    incl = x;
    u1 = u0 + __builtin_amdgcn_readlane(x, 63);
    return true;
  }

  // Units of the whole launch: the first group's prefix sum when it holds
  // every request (and n_wide: the units of its requests with more than 128
  // rows, whose blocks are wide), else a count over all requests.
  __device__ __forceinline__ int count_units(const AttnParams& p, int lane) {
    if (p.num_reqs <= 64) {
      if (!scan_group(p, lane)) return 0;
      const int r = lane;
      int wide = 0;
      if (r < p.num_reqs) {
        const int q_len = p.qsl[r + 1] - p.qsl[r];
        if (q_len * p.group > 2 * kBlockRows / 4)
          wide = request_row_tiles(q_len, p.blk_tok) * p.num_kv_heads;
      }
#pragma unroll
      for (int dd = 32; dd >= 1; dd >>= 1) wide += __shfl_xor(wide, dd);
      n_wide = __builtin_amdgcn_readfirstlane(wide);
      return u1;
    }
    int n = 0;
    for (int g = 0; g < p.num_reqs; g += 64) {
      const int r = g + lane;
      int tiles = r < p.num_reqs ? request_row_tiles(p.qsl[r + 1] - p.qsl[r], p.blk_tok) : 0;
#pragma unroll
      for (int dd = 32; dd >= 1; dd >>= 1) tiles += __shfl_xor(tiles, dd);
      n += __builtin_amdgcn_readfirstlane(tiles);
    }
    return n * p.num_kv_heads;
  }

  __device__ __forceinline__ bool next(const AttnParams& p, int lane, Block& B) {
    const int W = gridDim.x;
    const int b = blockIdx.x;
    const int H = p.num_kv_heads;
    const int M = W % H == 0 ? W / H : 0;
    // The work-group's slot in a decode round: slot H t + h (KV head h of the
    // round's t-th row tile) is work-group h M + t (M = W / H); with M a
    // multiple of 8 (a full grid of 256) the H heads of a row tile run on one
    // XCD.
    const int slot = M > 0 ? (b % M) * H + b / M : b;
    if (total < 0) {
      total = count_units(p, lane);
      nrounds = (total + W - 1) / W;
      rot = nrounds > 1 ? (b % 8) % nrounds : 0;
    }
    int u;
    do {
      if (round >= nrounds) return false;
      const int rr = round + rot < nrounds ? round + rot : round + rot - nrounds;
      ++round;
      // Rounds of wide blocks (prefill): slot b, so that the row tiles of one
      // KV head, which read the same keys, share an XCD's L2.
      const int sl = rr * W < n_wide ? b : slot;
      u = rr * W + ((rr & 1) ? W - 1 - sl : sl);
    } while (u >= total);
    if (u < u0) {  // a wrapped round: scan again from the first group
      r0 = -64;
      u0 = u1 = 0;
    }
    while (u >= u1)
      if (!scan_group(p, lane)) return false;
    const int local = u - u0;
    const int j = static_cast<int>(__popcll(__ballot(incl <= local)));
    const int req = r0 + __builtin_amdgcn_readlane(sreq, j);
    const int u_loc = local - (j > 0 ? __builtin_amdgcn_readlane(incl, j - 1) : 0);
    const int q_start = ld_ro(p.qsl, req);
    const int q_len = ld_ro(p.qsl, req + 1) - q_start;
    const int seq_len = ld_ro(p.seq_lens, req);
    const int nb = request_row_tiles(q_len, p.blk_tok);
    const int jb = u_loc / p.num_kv_heads;
    const int kvh = u_loc - jb * p.num_kv_heads;
    const RowTile t = request_tile(req, q_start, q_len, seq_len, p.blk_tok, nb - 1 - jb);
    make_block<kWindow>(p, t, kvh, B);
    return true;
  }
};

// The 32 rows [row0, row0 + 32) of a block as one wave sees them.
struct RowSet {
  bool has_rows;
  bool two;                // rows row0 + 16 .. exist
  int w_lo_min, w_lo_max;  // key_lo over the rows
  int w_hi_min, w_hi_max;  // key_hi over the rows
};

template <bool kWindow>
__device__ __forceinline__ RowSet make_rowset(const AttnParams& p, const Block& B, int row0) {
  const int window = kWindow ? p.window : 0;
  const bool causal = kWindow ? (p.causal != 0) : true;
  RowSet R;
  const int n = B.rows - row0;
  R.has_rows = n > 0;
  R.two = n > kRowsPerWave;
  R.w_lo_min = R.w_lo_max = 0;
  R.w_hi_min = R.w_hi_max = -1;
  if (!R.has_rows) return R;
  const int last = row0 + (n < kWaveRows ? n : kWaveRows) - 1;
  const int tok_first = B.t.tok_begin + static_cast<int>(p.g_div.div(row0));
  const int tok_last = B.t.tok_begin + static_cast<int>(p.g_div.div(last));
  R.w_lo_min = key_lo(B.t, tok_first, window);
  R.w_lo_max = key_lo(B.t, tok_last, window);
  R.w_hi_min = key_hi(B.t, tok_first, window, causal);
  R.w_hi_max = key_hi(B.t, tok_last, window, causal);
  return R;
}

// A 16-row group of the block as a Unit (for unit_lanes and finish).
__device__ __forceinline__ Unit group_unit(const Block& B, int row0) {
  Unit U;
  U.t = B.t;
  U.s = 0;
  U.live = 1;
  U.kvh = B.kvh;
  U.rg = 0;
  U.rows = B.rows;
  U.row0 = row0;
  U.has_rows = row0 < B.rows;
  return U;
}

// Loads of the block's chunks: per-lane offsets of the KV head's cells (as
// the paged producer of attn_fwd.hip), and the pages of the next chunk to
// issue, looked up one chunk ahead so that an issue never waits for the
// block table.
struct RowLoader {
  uint32_t off_k[2], off_v[2], off_s;
  int64_t bt0;
  int32_t page[2], slot0[2];
};

__device__ __forceinline__ void row_loader(const AttnParams& p, const Block& B, int lane,
                                           RowLoader& Ld) {
  const uint32_t kq = lane >> 3, piece = lane & 7;
  const uint32_t head = static_cast<uint32_t>(B.kvh) * p.cell_head;
  const uint32_t sw = 16u * (piece ^ kq);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t row = (8u * h + kq) * p.cell_slot + head + sw;
    Ld.off_k[h] = row + p.cell_off[0];
    Ld.off_v[h] = row + p.cell_off[1];
  }
  Ld.off_s = static_cast<uint32_t>(lane & 15) * p.cell_slot + head +
             (lane < 32 ? p.cell_off[2] : p.cell_off[3]);
  Ld.bt0 = static_cast<int64_t>(B.t.req) * p.bt_stride;
}

// Block-table windows of a key part (the parts path): each wave keeps 64
// consecutive entries of its request's block-table row, from block
// wb0 + 64 w, in LDS (two buffers: window w and w + 1), loaded with one
// direct-to-LDS dword load per lane. A chunk's pages are then two LDS reads,
// where a scalar load of the block table per chunk made each step wait with
// lgkmcnt(0) (a scalar load completes out of order, so its wait covers every
// later LDS and scalar operation too); config 5 4.72 -> 4.61 ms with the
// head-grouped rotation.
// Window w + 1 is loaded when window w comes into use, at least 32 chunks
// (64 blocks of >= 16 keys) before its first use: the chunk waits in between
// (vmcnt, in-order completion) cover its load. The extra loads only make
// those waits count one operation too few, that is wait longer, never less.
constexpr int kBtWindow = 64;                          // entries per window
constexpr int kBtWaveBytes = 2 * kBtWindow * 4;        // two windows per wave
constexpr int kBtBase = kRowSlots * kSlotBytes;        // after the chunk slots
constexpr int kRowLds = kBtBase + kRowWaves * kBtWaveBytes;
static_assert(kRowLds <= 160 * 1024, "row-block kernel LDS");

struct BtWindows {
  int wb0;       // first block of window 0
  int wi;        // the current window
  int last_blk;  // last block a load may read (inside the request's row)
};

// Window w of the wave's buffers `bt` (lane l: entry min(wb0 + 64 w + l,
// last_blk) of the row).
__device__ __forceinline__ void bt_window_load(const AttnParams& p, const RowLoader& Ld,
                                               const BtWindows& W, int w, char* bt, int lane) {
  int e = W.wb0 + kBtWindow * w + lane;
  e = e < W.last_blk ? e : W.last_blk;
  dma4(reinterpret_cast<const char*>(p.block_table + Ld.bt0 + e), bt + (w & 1) * (kBtWindow * 4));
}

// Windows 0 and 1 of a part whose keys start at c0 (issued before the
// vmcnt(0) that waits for the query).
__device__ __forceinline__ void bt_windows_start(const AttnParams& p, const Block& B,
                                                 const RowLoader& Ld, int c0, BtWindows& W,
                                                 char* bt, int lane) {
  const int first = c0 > B.ld_lo ? c0 : B.ld_lo;
  W.wb0 = static_cast<int>(p.bs_div.div(first));
  W.wi = 0;
  W.last_blk = static_cast<int>(p.bs_div.div(B.ld_hi > 0 ? B.ld_hi - 1 : 0));
  bt_window_load(p, Ld, W, 0, bt, lane);
  bt_window_load(p, Ld, W, 1, bt, lane);
}

// Pages of the chunk at key c from the windows (a 16-key group outside the
// block's keys gets page 0, masked later). Blocks only move forward, so a
// block past window wi + 1 never occurs before window wi + 1 is current.
__device__ __forceinline__ void rows_pages(const AttnParams& p, const Block& B, int c,
                                           RowLoader& Ld, BtWindows& W, char* bt,
                                           uint32_t bt_lds, int lane) {
  bool use[2];
  int blk[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int c16 = c + 16 * sub;
    use[sub] = c16 < B.ld_hi && c16 + 16 > B.ld_lo;
    blk[sub] = use[sub] ? static_cast<int>(p.bs_div.div(c16)) : W.wb0;
    Ld.slot0[sub] = use[sub] ? c16 - blk[sub] * static_cast<int>(p.bs_div.d) : 0;
  }
  const int b0 = use[0] ? blk[0] : blk[1];
  if (use[0] || use[1]) {
    const int need = (b0 - W.wb0) >> 6;
    if (need > W.wi) {  // window wi + 1 becomes current; load wi + 2
      ++W.wi;
      bt_window_load(p, Ld, W, W.wi + 1, bt, lane);
    }
  }
  float e[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int d = blk[sub] - W.wb0;
    e[sub] = ds_read4(bt_lds + (((d >> 6) & 1) * kBtWindow + (d & 63)) * 4);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(e[0]), "+v"(e[1]) : : "memory");
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    Ld.page[sub] = use[sub] ? __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, e[sub])) : 0;
}

// This wave's share of the 9 loads of the chunk whose pages Ld holds: loads
// d with d % RS == rs (d < 4: K rows 8d .. 8d + 7; d < 8: V rows
// 8(d - 4) ..; d = 8: the 64 scales), laid out as the paged producer of
// attn_fwd.hip lays them out.
__device__ __forceinline__ void issue_rows_chunk(const AttnParams& p, const RowLoader& Ld,
                                                 char* slot, int rs, int mask, int lane) {
  const char* base[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
    base[sub] = p.cell_base +
                static_cast<uint64_t>(static_cast<uint32_t>(Ld.page[sub])) * p.cell_block +
                static_cast<uint32_t>(Ld.slot0[sub]) * p.cell_slot;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if ((d & mask) == rs) dma16(base[d >> 1] + Ld.off_k[d & 1], slot + kSlotK + 1024 * d);
    if (((d + 4) & mask) == rs) dma16(base[d >> 1] + Ld.off_v[d & 1], slot + kSlotV + 1024 * d);
  }
  if ((8 & mask) == rs) dma4(((lane >> 4) & 1 ? base[1] : base[0]) + Ld.off_s, slot + kSlotScale);
}

// Loads per chunk issued by row set rs of RS = mask + 1.
__device__ __forceinline__ int rows_chunk_loads(int mask, int rs) {
  int n = 0;
#pragma unroll
  for (int d = 0; d < kDmaPerChunk; ++d) n += (d & mask) == rs ? 1 : 0;
  return n;
}

// One 32-key chunk at key c for the wave's two 16-row groups: compute_chunk
// of attn_device.h, each K and V operand used by both groups. `ops` gives
// the bf16 operands (converted from the int8 chunk, or read from the
// work-group's converted copy): ops.sc() the lane's scale, ops.k(sub, j),
// ops.load_v() (issued before the softmax) and ops.v(j).
// kBoth: compute both groups whether or not the second has rows (the wide
// path: group 1 of a wave without rows repeats group 0 and is dropped). No
// branch then separates the MFMAs (-5 % on a mixed prefill launch).
template <bool kF16Q, bool kBoth, class Ops>
__device__ __forceinline__ void compute_rows(const RowSet& R, const Lanes (&L)[2], int c, Ops& ops,
                                             const bf16x8 (&qb)[2][4], const bf16x8 (&qlo)[2][4],
                                             float scl, State (&st)[2], int& vexp, float& vlim) {
  float ks[8], vs[8];
  ops.scales(scl, ks, vs);
  const int ng = kBoth || R.two ? 2 : 1;
  bool fresh[2];
  float m_use[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    fresh[i] = st[i].m == kNegInf;
    m_use[i] = fresh[i] ? 0.0f : st[i].m;
  }
  float t[2][8];
  // The QK MFMAs run at raised wave priority: the SIMD's other wave, in its
  // softmax, fills the VALU slots between them (measured -2.5 % on a mixed
  // prefill launch; raising it for the PV products as well gained nothing).
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8 a = ops.k(sub, j);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (i < ng) {
          acc[i] = mfma(a, qb[i][j], acc[i]);
          if constexpr (kF16Q) acc[i] = mfma(a, qlo[i][j], acc[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        t[i][4 * sub + e] = fmaf(acc[i][e], ks[4 * sub + e], -m_use[i]);
  }
  // Waves 4-7 keep priority 1 for the whole block (see attn_fwd_rows).
  if ((__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x)) >> 8) == 0)
    __builtin_amdgcn_s_setprio(0);
  ops.load_v();
  if (c < R.w_lo_max || c + kChunkTokens - 1 > R.w_hi_min) {
    // Keys outside a row's range get p = 0; keys outside every row's range
    // (possibly outside the request: any bits, a scale included) also a zero
    // V scale. Keys inside some row's range are cache data of the request.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = c + 16 * (e >> 2) + 4 * L[0].g + (e & 3);
      if (key < R.w_lo_min || key > R.w_hi_max) vs[e] = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (key < L[i].lo || key > L[i].hi) t[i][e] = kNegInf;
    }
  }
  // The V scales times 2^-C (C: the running exponent; every V scale seen so
  // far is below 2^C), so that p vs 2^-C < 2^8 fits fp16; O is kept in units
  // of 2^-C and rescaled when C grows (undo_vexp folds 2^C back in).
  if constexpr (Ops::kNormalised) {
    const int e = ops.vexp();  // normalised by the converting wave
    if (e > vexp) {
      if (vexp != kNoExp) {
        const float f = __builtin_ldexpf(1.0f, vexp - e);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 8; ++j) st[i].o[j] *= f;
      }
      vexp = e;
    }
  } else {
    // A V scale of this chunk at or above 2^C (masked keys have 0): raise C
    // to the chunk's largest.
    if (__ballot(max8_raw(vs) >= vlim) != 0) {
      const int e = vscale_exp(xor_max(max8_raw(vs)));
      if (e > vexp) {
        if (vexp != kNoExp) {
          const float f = __builtin_ldexpf(1.0f, vexp - e);
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) st[i].o[j] *= f;
        }
        vexp = e;
        vlim = __builtin_ldexpf(1.0f, e);
      }
    }
    const float vnorm = __builtin_ldexpf(1.0f, vexp == kNoExp ? 0 : -vexp);
#pragma unroll
    for (int e2 = 0; e2 < 8; ++e2) vs[e2] *= vnorm;
  }
  f16x8 p16[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (i >= ng) continue;
    // A row's max exceeds the threshold iff one of its 4 lanes' maxima does:
    // the cross-lane reduction runs only when some row grows.
    const float lane_mx = max8_raw(t[i]);
    if (__ballot(lane_mx > rescale_threshold(fresh[i])) != 0) {
      const float mx = xor_max(lane_mx);
      const bool grow = mx > rescale_threshold(fresh[i]);
      const float alpha = grow && !fresh[i] ? __builtin_amdgcn_exp2f(-mx) : 1.0f;
      st[i].l *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) st[i].o[j] *= alpha;
      const float shift = grow ? mx : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[i][e] -= shift;
      st[i].m = grow ? m_use[i] + mx : st[i].m;
    }
    float pv[8];
    float lsum;  // the sum starts at the first term (an added 0 is an instruction)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pe = __builtin_amdgcn_exp2f(t[i][e]);
      lsum = e == 0 ? pe : lsum + pe;
      pv[e] = pe * vs[e];
    }
    st[i].l += lsum;
#pragma unroll
    for (int e = 0; e < 8; ++e) p16[i][e] = static_cast<_Float16>(pv[e]);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const f16x8 vcol = ops.v(j);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (i < ng) st[i].o[j] = mfma_f16(vcol, p16[i], st[i].o[j]);
  }
}

// ---------------------------------------------------------------------------
// Wide blocks (one key part: all 8 waves compute every chunk). The int8 ->
// bf16 / fp16 conversion is shared: each wave converts one eighth of a chunk
// into a copy in LDS, one chunk ahead of the compute, and every wave reads its
// MFMA operands from the copy. Copy layout (16 KB, lane-contiguous):
//   K: [sub 2][j 4][lane 64] x 16 B  -- bf16 K[16 sub + (l % 16)][32 (l / 16) + 8 j ..]
//   V: [j 8][lane 64] x 16 B         -- fp16 V[tv(e)][8 (l % 16) + j], e = 0..7
// Wave w converts K operand (sub, j) = (w / 4, w % 4) and V column j = w.
// A wide block advances two chunks per barrier step: step s computes chunks
// 2s, 2s + 1, converts chunks 2s + 2, 2s + 3 and issues the loads of chunks
// 2s + 6, 2s + 7 (so four chunks are in flight), into the int8 slots that
// chunks 2s - 2, 2s - 1 left.
constexpr int kWideSlots = 8;  // int8 chunk slots of a wide block
constexpr int kCopyBytes = 16384;
constexpr int kCopies = 4;     // copies: the pair computed and the pair converted
constexpr int kCopyBase = kWideSlots * kSlotBytes;
// The exponent C each copy's V scales were normalised by (one int per copy).
constexpr int kCopyExp = kCopyBase + kCopies * kCopyBytes;
static_assert(kCopyExp + 4 * kCopies <= kRowSlots * kSlotBytes, "wide-block LDS");

template <int kOff>
__device__ __forceinline__ uint32_t ds_read_i8(uint32_t a) {
  uint32_t v;
  asm volatile("ds_read_i8 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(kOff));
  return v;
}
__device__ __forceinline__ void ds_write4(uint32_t a, float v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory");
}
template <int kOff>
__device__ __forceinline__ void ds_write16(uint32_t a, u32x4 v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(a), "v"(v), "n"(kOff) : "memory");
}

template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               kCtrl, 0xf, 0xf, false));
}
// Max over each row of 16 lanes (DPP; every lane of the row gets it).
__device__ __forceinline__ float wave_max16(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = fmaxf(x, dpp_mov<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = fmaxf(x, dpp_mov<0x141>(x));  // row_half_mirror
  return fmaxf(x, dpp_mov<0x140>(x));  // row_mirror
}

// Per-lane LDS offsets of the conversion reads (chunk slot relative).
struct ConvOffsets {
  uint32_t k;     // 8 bytes of K
  uint32_t v[4];  // byte j of the V run of key 4g + q (+ 2048: key 16 + 4g + q)
};

__device__ __forceinline__ ConvOffsets conv_offsets(int wave, int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const int sub = wave >> 2, j = wave & 3;
  ConvOffsets o;
  o.k = kSlotK + swz(16 * sub + r16, 2 * g + (j >> 1)) + 8 * (j & 1);
#pragma unroll
  for (int q = 0; q < 4; ++q) o.v[q] = kSlotV + swz(4 * g + q, r16 >> 1) + 8 * (r16 & 1) + wave;
  return o;
}

// The running V-scale exponent of a wide block's chunks, kept by its
// converting wave: every V scale of the block's keys converted so far is
// below lim = 2^exp (lim = 0 before the first).
struct VScaleBound {
  int exp = kNoExp;
  float lim = 0.0f;
};

// Wave `wave`'s eighth of the chunk in int8 slot `slot` -> copy `copy` (K in
// bf16, V in fp16). The last wave also prepares the chunk's scales in place:
// the K scales times scale * log2 e (the product the chunk step would form
// per lane), the V scales times 2^-C with C = vb.exp after this chunk (keys
// outside [ld_lo, ld_hi) are masked by every row and do not count), and
// writes C to `cslot` for the computing waves (vbd: the block's bound).
__device__ __forceinline__ void convert_share(uint32_t slot, uint32_t copy, const ConvOffsets& o,
                                              float scale_log2, int wave, int lane, int key0,
                                              int ld_lo, int ld_hi, VScaleBound& vbd,
                                              uint32_t cslot) {
  if (wave == kRowWaves - 1) {
    const uint32_t sa = slot + kSlotScale + 4 * lane;  // K scales, then V scales
    float x = ds_read4(sa);
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x) : : "memory");
    const int key = key0 + (lane & (kChunkTokens - 1));
    const float v = lane >= kChunkTokens && key >= ld_lo && key < ld_hi ? x : 0.0f;
    if (__ballot(v >= vbd.lim) != 0) {  // a scale at or above the bound: raise it
      const int e = vscale_exp(xor_max(wave_max16(v)));
      if (e > vbd.exp) {
        vbd.exp = e;
        vbd.lim = __builtin_ldexpf(1.0f, e);
      }
    }
    ds_write4(sa, lane < kChunkTokens ? x * scale_log2
                                      : x * __builtin_ldexpf(1.0f, vbd.exp == kNoExp ? 0 : -vbd.exp));
    if (lane == 0) asm volatile("ds_write_b32 %0, %1" ::"v"(cslot), "v"(vbd.exp) : "memory");
  }
  u32x2 kw = ds_read8<0>(slot + o.k);
  uint32_t vb[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    vb[q] = ds_read_i8<0>(slot + o.v[q]);
    vb[4 + q] = ds_read_i8<2048>(slot + o.v[q]);
  }
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(kw), "+v"(vb[0]), "+v"(vb[1]), "+v"(vb[2]), "+v"(vb[3]), "+v"(vb[4]),
                 "+v"(vb[5]), "+v"(vb[6]), "+v"(vb[7])
               :
               : "memory");
  const bf16x8 ka = i8x8_to_bf16(kw[0], kw[1]);
  // V column: the 8 keys in e order (tv(e) = 16 (e / 4) + 4 g + e % 4).
  // Keys e, e + 1 into the low and high halves of one dword: int16 -> fp16,
  // exact, the second through SDWA into the upper word (one instruction per
  // value; the compiler's form converts and then packs).
  u32x4 vp;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t w;
    asm("v_cvt_f16_i16_e32 %0, %1\n\t"
        "v_cvt_f16_i16_sdwa %0, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0"
        : "=&v"(w)
        : "v"(vb[2 * d]), "v"(vb[2 * d + 1]));
    vp[d] = w;
  }
  const f16x8 va = __builtin_bit_cast(f16x8, vp);
  const uint32_t dst = copy + wave * 1024 + lane * 16;
  ds_write16<0>(dst, __builtin_bit_cast(u32x4, ka));
  ds_write16<8192>(dst, __builtin_bit_cast(u32x4, va));
}

// Operands of compute_rows from the int8 chunk in registers.
struct Int8Ops {
  static constexpr bool kNormalised = false;  // V scales as stored: the wave normalises
  const Chunk& ch;
  __device__ __forceinline__ void scales(float scl, float (&ks)[8], float (&vs)[8]) const {
    lane_scales(ch.sc * scl, ks, vs);
  }
  __device__ __forceinline__ bf16x8 k(int sub, int j) const {
    const u32x4& w = ch.k[sub][j >> 1];
    return (j & 1) ? i8x8_to_bf16(w[2], w[3]) : i8x8_to_bf16(w[0], w[1]);
  }
  __device__ __forceinline__ void load_v() const {}
  __device__ __forceinline__ f16x8 v(int j) const { return column_to_f16(ch.v, j); }
};

// Operands of compute_rows from a converted copy: K and the scales read at
// construction, V read by load_v. The chunk's K scales in its int8 slot were
// multiplied by scale * log2 e when it was converted (convert_share), so a
// lane reads its 8 K and 8 V scales as they are: keys 4 g .. 4 g + 3 and
// 16 + 4 g .., four 16-byte reads that the 16 lanes of a row share.
struct CopyOps {
  static constexpr bool kNormalised = true;  // V scales times 2^-vexp() (convert_share)
  uint32_t a;  // copy + 16 lane
  u32x4 kk[8];
  u32x4 vv[8];
  u32x4 sk[2], sv[2];

  int cexp;    // the exponent the chunk's V scales were normalised by

  __device__ __forceinline__ int vexp() const { return cexp; }
  __device__ __forceinline__ CopyOps(uint32_t copy, uint32_t slot, uint32_t cslot, int lane)
      : a(copy + lane * 16) {
    uint32_t ce;
    asm volatile("ds_read_b32 %0, %1" : "=v"(ce) : "v"(cslot));
    const uint32_t sa = slot + kSlotScale + 16 * (lane >> 4);
    sk[0] = ds_read16<0>(sa);
    sk[1] = ds_read16<64>(sa);
    sv[0] = ds_read16<128>(sa);
    sv[1] = ds_read16<192>(sa);
    kk[0] = ds_read16<0>(a);
    kk[1] = ds_read16<1024>(a);
    kk[2] = ds_read16<2048>(a);
    kk[3] = ds_read16<3072>(a);
    kk[4] = ds_read16<4096>(a);
    kk[5] = ds_read16<5120>(a);
    kk[6] = ds_read16<6144>(a);
    kk[7] = ds_read16<7168>(a);
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(kk[0]), "+v"(kk[1]), "+v"(kk[2]), "+v"(kk[3]), "+v"(kk[4]), "+v"(kk[5]),
                   "+v"(kk[6]), "+v"(kk[7]), "+v"(sk[0]), "+v"(sk[1]), "+v"(sv[0]), "+v"(sv[1]),
                   "+v"(ce)
                 :
                 : "memory");
    cexp = __builtin_amdgcn_readfirstlane(static_cast<int>(ce));
  }
  __device__ __forceinline__ void scales(float, float (&ks)[8], float (&vs)[8]) const {
    // Each element goes through a named scalar: a bit cast of a subscripted
    // vector element reads element 0 with this compiler.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t kw = sk[e >> 2][e & 3], vw = sv[e >> 2][e & 3];
      ks[e] = __builtin_bit_cast(float, kw);
      vs[e] = __builtin_bit_cast(float, vw);
    }
  }
  __device__ __forceinline__ bf16x8 k(int sub, int j) const {
    return __builtin_bit_cast(bf16x8, kk[4 * sub + j]);
  }
  __device__ __forceinline__ void load_v() {
    vv[0] = ds_read16<8192>(a);
    vv[1] = ds_read16<9216>(a);
    vv[2] = ds_read16<10240>(a);
    vv[3] = ds_read16<11264>(a);
    vv[4] = ds_read16<12288>(a);
    vv[5] = ds_read16<13312>(a);
    vv[6] = ds_read16<14336>(a);
    vv[7] = ds_read16<15360>(a);
  }
  // The first use waits for all eight (the softmax in between hides the
  // LDS latency).
  __device__ __forceinline__ f16x8 v(int j) {
    if (j == 0)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(vv[0]), "+v"(vv[1]), "+v"(vv[2]), "+v"(vv[3]), "+v"(vv[4]),
                     "+v"(vv[5]), "+v"(vv[6]), "+v"(vv[7])
                   :
                   : "memory");
    return __builtin_bit_cast(f16x8, vv[j]);
  }
};

// Merge area of writer w (a wave of key part >= 1): O, m, l per lane.
__device__ __forceinline__ char* merge_area(char* lds, int w) { return lds + w * kMergeBytes; }

// (Loops over the two groups are unrolled with constant indices: a
// run-time index would move the states to scratch memory.)
__device__ __forceinline__ void merge_store(char* a, int lane, const State (&st)[2], int ng) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (i >= ng) break;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<f32x4*>(a + ((i * 8 + j) * 64 + lane) * 16) = st[i].o[j];
    *reinterpret_cast<float*>(a + kMergeO + (i * 64 + lane) * 4) = st[i].m;
    *reinterpret_cast<float*>(a + kMergeO + 512 + (i * 64 + lane) * 4) = st[i].l;
  }
}

// st := st (+) the partial of area a: the same rows, another part of the keys.
__device__ __forceinline__ void merge_add(const char* a, int lane, State& st, int i) {
  const float mj = *reinterpret_cast<const float*>(a + kMergeO + (i * 64 + lane) * 4);
  const float lj = *reinterpret_cast<const float*>(a + kMergeO + 512 + (i * 64 + lane) * 4);
  const float M = fmaxf(st.m, mj);
  if (M == kNegInf) return;  // neither part has seen a key of this row
  const float a0 = __builtin_amdgcn_exp2f(st.m - M);
  const float a1 = __builtin_amdgcn_exp2f(mj - M);
  st.l = st.l * a0 + lj * a1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const f32x4 oj = *reinterpret_cast<const f32x4*>(a + ((i * 8 + j) * 64 + lane) * 16);
    st.o[j] = st.o[j] * a0 + oj * a1;
  }
  st.m = M;
}

// Pages of the two chunks at key c (4 groups of 16 keys), looked up one step
// ahead of their loads.
struct PairPages {
  int32_t page[4], slot0[4];
};

__device__ __forceinline__ void pair_pages(const AttnParams& p, const Block& B, int64_t bt0, int c,
                                           PairPages& pp) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c16 = c + 16 * q;
    pp.page[q] = 0;
    pp.slot0[q] = 0;
    if (c16 < B.ld_hi && c16 + 16 > B.ld_lo) {
      const int blk = static_cast<int>(p.bs_div.div(c16));
      pp.slot0[q] = c16 - blk * static_cast<int>(p.bs_div.d);
      pp.page[q] = ld_ro(p.block_table, bt0 + blk);
    }
  }
}

// Wave w's loads of chunk h (0, 1) of a pair: load d = w of the chunk (K rows
// 8w .. for w < 4, V rows 8(w - 4) .. otherwise), and wave 0 also the scales.
// The selection is wave-uniform arithmetic, no branch but the scales'.
__device__ __forceinline__ void issue_wide(const AttnParams& p, const RowLoader& Ld,
                                           const PairPages& pp, int h, char* slot, int wave,
                                           int lane) {
  const int q = wave & 3;
  const bool isv = wave >= 4;
  // Group 2h + (q >> 1), selected without indexing (a run-time index would
  // move the array to memory).
  const bool hi = (q >> 1) != 0;
  const int32_t page = h == 0 ? (hi ? pp.page[1] : pp.page[0]) : (hi ? pp.page[3] : pp.page[2]);
  const int32_t slot0 = h == 0 ? (hi ? pp.slot0[1] : pp.slot0[0]) : (hi ? pp.slot0[3] : pp.slot0[2]);
  const char* base = p.cell_base + static_cast<uint64_t>(static_cast<uint32_t>(page)) * p.cell_block +
                     static_cast<uint32_t>(slot0) * p.cell_slot;
  // Rows 8 (q & 1) + lane / 8 of the group, K or V: the lane's K offset of
  // the first row plus uniform terms (no selection between the offsets).
  const uint32_t off = Ld.off_k[0] + (isv ? p.cell_off[1] - p.cell_off[0] : 0u) +
                       static_cast<uint32_t>(q & 1) * 8u * p.cell_slot;
  dma16(base + off, slot + (isv ? kSlotV : kSlotK) + 1024 * q);
  if (wave == 0) {
    const int32_t pa = h == 0 ? pp.page[0] : pp.page[2], pb = h == 0 ? pp.page[1] : pp.page[3];
    const int32_t sa = h == 0 ? pp.slot0[0] : pp.slot0[2], sb = h == 0 ? pp.slot0[1] : pp.slot0[3];
    const char* b0 = p.cell_base + static_cast<uint64_t>(static_cast<uint32_t>(pa)) * p.cell_block +
                     static_cast<uint32_t>(sa) * p.cell_slot;
    const char* b1 = p.cell_base + static_cast<uint64_t>(static_cast<uint32_t>(pb)) * p.cell_block +
                     static_cast<uint32_t>(sb) * p.cell_slot;
    dma4(((lane >> 4) & 1 ? b1 : b0) + Ld.off_s, slot + kSlotScale);
  }
}

// The chunk loop of a wide block, two chunks per step (see kWideSlots).
// Before step s the copies of chunks 2s, 2s + 1 are complete. Step s: wait
// for this wave's loads of chunks 2s + 2, 2s + 3; barrier (they are in LDS,
// every wave is done with step s - 1); issue chunks 2s + 6, 2s + 7; convert
// this wave's shares of chunks 2s + 2, 2s + 3; compute chunks 2s, 2s + 1.
template <bool kF16Q>
__device__ __forceinline__ void wide_block(const AttnParams& p, const Block& B, const RowSet& R,
                                           const Lanes (&L)[2], RowLoader& Ld,
                                           const bf16x8 (&qb)[2][4], const bf16x8 (&qlo)[2][4],
                                           float scl, State (&st)[2], char* lds, uint32_t lds_base,
                                           const ReadOffsets& ro, const ConvOffsets& cvo,
                                           int wave, int lane) {
  const int len = B.n_chunks;
  if (len == 0) return;
  int vexp = kNoExp;  // this wave's
  float vlim = 0.0f;  // (unused with the converted copies)
  VScaleBound vb;     // the converting wave's
  auto cslot = [&](int k) { return lds_base + kCopyExp + 4 * (k % kCopies); };
  const int nload = wave == 0 ? 2 : 1;
  const uint32_t copy0 = lds_base + kCopyBase;
  auto slot_of = [&](int k) { return (k % kWideSlots) * kSlotBytes; };
  auto copy_of = [&](int k) { return (k % kCopies) * kCopyBytes; };
  auto chunk_key = [&](int k) { return B.c_begin + kChunkTokens * k; };
  PairPages pp;
  for (int k = 0; k < 6 && k < len; k += 2) {
    pair_pages(p, B, Ld.bt0, chunk_key(k), pp);
    issue_wide(p, Ld, pp, 0, lds + slot_of(k), wave, lane);
    if (k + 1 < len) issue_wide(p, Ld, pp, 1, lds + slot_of(k + 1), wave, lane);
  }
  if (6 < len) pair_pages(p, B, Ld.bt0, chunk_key(6), pp);
  // Chunks 0, 1 landed: at most the loads of chunks 2 .. 5 outstanding.
  {
    const int issued = len < 6 ? len : 6;
    const int younger = issued - 2 > 0 ? issued - 2 : 0;
    wait_vmcnt_dyn(nload * younger);
  }
  wg_barrier();
  convert_share(lds_base + slot_of(0), copy0 + copy_of(0), cvo, p.scale_log2, wave, lane,
                chunk_key(0), B.ld_lo, B.ld_hi, vb, cslot(0));
  if (1 < len)
    convert_share(lds_base + slot_of(1), copy0 + copy_of(1), cvo, p.scale_log2, wave, lane,
                  chunk_key(1), B.ld_lo, B.ld_hi, vb, cslot(1));
  for (int k = 0; k < len; k += 2) {
    if (k + 2 < len) {
      // Issued so far: chunks up to min(k + 5, len - 1); k + 2, k + 3 must land.
      const int last = k + 5 < len - 1 ? k + 5 : len - 1;
      const int younger = last - (k + 3) > 0 ? last - (k + 3) : 0;
      wait_vmcnt_dyn(nload * younger);
    }
    wait_lgkmcnt0();  // this wave's copy writes
    wg_barrier();
    if (k + 6 < len) {
      issue_wide(p, Ld, pp, 0, lds + slot_of(k + 6), wave, lane);
      if (k + 7 < len) issue_wide(p, Ld, pp, 1, lds + slot_of(k + 7), wave, lane);
    }
    if (k + 2 < len)
      convert_share(lds_base + slot_of(k + 2), copy0 + copy_of(k + 2), cvo, p.scale_log2, wave,
                    lane, chunk_key(k + 2), B.ld_lo, B.ld_hi, vb, cslot(k + 2));
    if (k + 3 < len)
      convert_share(lds_base + slot_of(k + 3), copy0 + copy_of(k + 3), cvo, p.scale_log2, wave,
                    lane, chunk_key(k + 3), B.ld_lo, B.ld_hi, vb, cslot(k + 3));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kk = k + h;
      const int c = chunk_key(kk);
      if (kk < len && R.has_rows && c <= R.w_hi_max && c + kChunkTokens > R.w_lo_min) {
        CopyOps ops(copy0 + copy_of(kk), lds_base + slot_of(kk), cslot(kk), lane);
        compute_rows<kF16Q, true>(R, L, c, ops, qb, qlo, scl, st, vexp, vlim);
      }
    }
    if (k + 8 < len) pair_pages(p, B, Ld.bt0, chunk_key(k + 8), pp);
  }
  undo_vexp(st[0], vexp);
  undo_vexp(st[1], vexp);
}

template <bool kWindow, bool kF16Q>
__global__ __launch_bounds__(kRowWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_rows(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) char lds[kRowLds];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lds_base = lds_offset(lds);
  const ReadOffsets ro = read_offsets(lane);
  const float scl = scale_factor(lane & 15, p.scale_log2);
  const ConvOffsets cvo = conv_offsets(wave, lane);
  BlockWalk<kWindow> walk;
  Block B;
  while (walk.next(p, lane, B)) {
    // The previous block's merge reads of the slots are done.
    __syncthreads();
    // Waves w and w + 4 share a SIMD, and between two barriers the arbiter's
    // preference for the older wave let waves 0-3 finish each step 0.5-0.8 us
    // before waves 4-7 and wait for them at the next barrier (per-step
    // timestamps, config 5's prefill part). Waves 4-7 therefore run the whole
    // block at priority 1, waves 0-3 only during their QK products
    // (compute_rows): the prefill part 4.05 -> 3.97 ms.
    if (wave >= kRowWaves / 2) __builtin_amdgcn_s_setprio(1);
    const int mask = (1 << B.log_rs) - 1;
    const int rs = wave & mask;
    const int part = wave >> B.log_rs;
    const int kp = B.kp;
    const int ns = kRowSlots / kp;
    // A part of one wave (RS == 1) owns its slots: it refills the slot it
    // has just read and needs no barrier, so its waves stream independently.
    // Parts of several waves refill a slot only after the barrier that
    // follows every wave's read of it.
    const bool solo = mask == 0;
    const int room = solo ? ns : ns - 1;
    const int ahead = kRowAhead < room ? kRowAhead : room;
    const int pc0 = part * B.n_chunks / kp;
    const int len = (part + 1) * B.n_chunks / kp - pc0;
    const int steps = (B.n_chunks + kp - 1) / kp;
    char* ring = lds + part * ns * kSlotBytes;
    const uint32_t ring_base = lds_base + part * ns * kSlotBytes;
    const int nload = rows_chunk_loads(mask, rs);

    const int row0 = rs * kWaveRows;
    const RowSet R = make_rowset<kWindow>(p, B, row0);
    const Unit U0 = group_unit(B, row0), U1 = group_unit(B, row0 + kRowsPerWave);
    Lanes L[2];
    L[0] = unit_lanes<kWindow>(p, U0, lane);
    L[1] = R.two ? unit_lanes<kWindow>(p, U1, lane) : L[0];
    RowLoader Ld;
    row_loader(p, B, lane, Ld);
    const int c0 = B.c_begin + kChunkTokens * pc0;
    char* bt = lds + kBtBase + wave * kBtWaveBytes;
    const uint32_t bt_lds = lds_base + kBtBase + wave * kBtWaveBytes;
    BtWindows btw;
    if (kp > 1 && len > 0) bt_windows_start(p, B, Ld, c0, btw, bt, lane);
    bf16x8 qb[2][4], qlo[2][4];
    if (R.has_rows) {
      load_q<kF16Q>(p, L[0], qb[0], qlo[0]);
      if (R.two) {
        load_q<kF16Q>(p, L[1], qb[1], qlo[1]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          qb[1][j] = qb[0][j];
          qlo[1][j] = qlo[0][j];
        }
      }
    }
    // Q (and the block-table windows) have landed (a compiler-visible
    // vmcnt(0): the chunk waits below are asm the compiler does not see).
    __builtin_amdgcn_s_waitcnt(0x0F70);
    State st[2];
    state_reset(st[0]);
    state_reset(st[1]);

    if (kp == 1) {
      wide_block<kF16Q>(p, B, R, L, Ld, qb, qlo, scl, st, lds, lds_base, ro, cvo, wave, lane);
      if (R.has_rows) {
        epilogue(p, U0, L[0], st[0]);
        if (R.two) epilogue(p, U1, L[1], st[1]);
      }
      continue;
    }
    if (len > 0) rows_pages(p, B, c0, Ld, btw, bt, bt_lds, lane);
    for (int i = 0; i < ahead && i < len; ++i) {
      issue_rows_chunk(p, Ld, ring + i * kSlotBytes, rs, mask, lane);
      if (i + 1 < len) rows_pages(p, B, c0 + kChunkTokens * (i + 1), Ld, btw, bt, bt_lds, lane);
    }
    const int nsteps = solo ? len : steps;
    int vexp = kNoExp;
    float vlim = 0.0f;  // 2^vexp (0: no V scale seen yet)
    for (int k = 0; k < nsteps; ++k) {
      if (k < len) {
        const int last = k + ahead - 1 < len - 1 ? k + ahead - 1 : len - 1;
        wait_vmcnt_dyn(nload * (last - k));
      }
      // After the barrier chunk k is complete in LDS and every wave is done
      // reading chunk k - 1.
      if (!solo) wg_barrier();
      const int c = c0 + kChunkTokens * k;
      const bool mine = k < len && R.has_rows && c <= R.w_hi_max && c + kChunkTokens > R.w_lo_min;
      Chunk ch;
      // Read before the issue below: its page lookup waits for the LDS
      // counter.
      if (mine) read_chunk(ring_base + (k % ns) * kSlotBytes, ro, ch);
      if (k + ahead < len) {
        issue_rows_chunk(p, Ld, ring + ((k + ahead) % ns) * kSlotBytes, rs, mask, lane);
        if (k + ahead + 1 < len)
          rows_pages(p, B, c + kChunkTokens * (ahead + 1), Ld, btw, bt, bt_lds, lane);
      }
      if (mine) {
        Int8Ops ops{ch};
        compute_rows<kF16Q, false>(R, L, c, ops, qb, qlo, scl, st, vexp, vlim);
      }
    }
    undo_vexp(st[0], vexp);
    undo_vexp(st[1], vexp);
    const int ng = R.two ? 2 : 1;
    if (kp > 1) {
      __syncthreads();  // every wave is done with the slots
      if (part > 0 && R.has_rows) merge_store(merge_area(lds, wave - (mask + 1)), lane, st, ng);
      __syncthreads();
      if (part == 0 && R.has_rows) {
        for (int j = 1; j < kp; ++j) {
          const char* a = merge_area(lds, (j - 1) * (mask + 1) + rs);
#pragma unroll
          for (int i = 0; i < 2; ++i)
            if (i < ng) merge_add(a, lane, st[i], i);
        }
      }
    }
    if (part == 0 && R.has_rows) {
      epilogue(p, U0, L[0], st[0]);
      if (R.two) epilogue(p, U1, L[1], st[1]);
    }
  }
}

}  // namespace

hipError_t launch_rows_kernel(const AttnParams& p, dim3 grid, bool windowed, bool q_f16,
                              hipStream_t stream) {
  const dim3 block(kRowWaves * 64);
  if (windowed) {
    if (q_f16) hipLaunchKernelGGL((attn_fwd_rows<true, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((attn_fwd_rows<true, false>), grid, block, 0, stream, p);
  } else {
    if (q_f16) hipLaunchKernelGGL((attn_fwd_rows<false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((attn_fwd_rows<false, false>), grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

int32_t rows_block_tokens(int32_t group) {
  return group >= kBlockRows ? 1 : kBlockRows / group;
}

}  // namespace pa
