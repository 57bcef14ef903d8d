// attn_combine.hip -- merge of the split-KV partials (flash-decoding
// combine), head size D = 64, 128 or 256.
//
// Split s of a query row left o_s (fp32, normalised) and lse_s = m_s +
// log2(l_s) (log2 units; -inf when the split saw no key). The exact output is
//   out = sum_s 2^lse_s o_s / sum_s 2^lse_s
// and with M = max over live splits it is computed as
//   out = sum_s w_s o_s / sum_s w_s,   w_s = 2^(lse_s - M) in (0, 1].
// Rules (reference combine_kernel.cuh:6-22, attn_args.h:38-44): M over live
// splits only; a -inf split contributes nothing and its o_s (possibly stale
// or uninitialised memory) never enters an arithmetic operation; the sums run
// in the fixed order s = 0..S-1, so the result is deterministic.
//
// Few rows with many splits (shared_rows): up to 512 splits, a work-group of
// 16 waves per (token, head) row and 32 of its columns (wave w merges split
// block w, wave 0 merges the 16 results in a fixed order); beyond 512, one
// work-group per row (wave w merges the 16-split blocks w, w + 16, ...).
// Otherwise one wave per row.
// The kernels are latency-bound, so the loads are ordered by round: the
// padding bound, the split-count marker and the wave's LSEs are issued
// together (the LSEs before their count is known; slots past it are then
// dropped), then the partial rows of every split with a nonzero weight.
// Lane l owns columns [l NC, (l + 1) NC), NC = D / 64, so a split's row is
// one coalesced 4 D-byte read. Lane s loads lse_s (64 splits per instruction);
// the weights are broadcast with readlane and the o loads of 16 splits are
// issued before their fused multiply-adds. On the op path (the launcher
// passes the request lengths) only the splits the attention kernel wrote for
// the row are read: their count is the marker the kernel left in the row's
// last LSE slot (attn_device.h), and a row with a single split is left as
// the attention kernel wrote it to out.

#include "attn_stream.h"

namespace pa {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_inff();
// Splits whose o loads are issued together (before their multiply-adds).
template <int NC>
constexpr int kBatch = 32 / NC;

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, dpp_i32<kCtrl>(__builtin_bit_cast(int, v)));
}
// Maximum over the 64 lanes (every lane; DPP within rows of 16 lanes, then
// the four row maxima).
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = fmaxf(x, dpp_f32<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = fmaxf(x, dpp_f32<0x141>(x));  // row_half_mirror
  x = fmaxf(x, dpp_f32<0x140>(x));  // row_mirror
  auto lane_f = [&](int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
  };
  return fmaxf(fmaxf(lane_f(0), lane_f(16)), fmaxf(lane_f(32), lane_f(48)));
}
// Butterfly sum: within each row of 16 lanes every lane adds the same pairs
// (commutatively; quad swaps, then half-row and row mirrors pair the quad and
// half-row sums), then the row sums as (r0 + r1) + (r2 + r3) -- the pairing
// of a butterfly over lane distances 1, 2, ..., 32, so every lane holds the
// same, order-fixed total.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  auto lane_f = [&](int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
  };
  return (lane_f(0) + lane_f(16)) + (lane_f(32) + lane_f(48));
}

// Request of token tok: the number of requests that end at or before it
// (num_reqs for a padding row beyond qsl[R]).
__device__ __forceinline__ int request_of_token(const CombineParams& c, int64_t tok, int lane) {
  int r = 0;
  for (int r0 = 0; r0 < c.num_reqs; r0 += 64) {
    const int k = r0 + lane;
    const bool before = k < c.num_reqs && c.qsl[k + 1] <= tok;
    const int n = static_cast<int>(__popcll(__ballot(before)));
    r += n;
    if (n < 64) break;
  }
  return r;
}

// The splits the attention kernel wrote for row (tok, head) of request r
// under the stream partition: their count (live).
__device__ __forceinline__ int row_live_splits(const CombineParams& c, int r, int64_t tok,
                                               int head, int lane) {
  const StreamDesc d{c.qsl, c.seq_lens, c.num_reqs, c.bq, c.window, c.causal, c.n_hg,
                     c.num_wg, c.num_splits};
  int64_t total;
  const int64_t per = stream_per(d, lane, total);
  const int q_start = ld_ro(c.qsl, r);
  const int q_len = ld_ro(c.qsl, r + 1) - q_start;
  const int seq_len = ld_ro(c.seq_lens, r);
  const int tok_in = static_cast<int>(tok) - q_start;
  const int j = tok_in / c.bq;
  const int row = (tok_in - j * c.bq) * c.group + head % c.group;
  const int hu = (head / c.group) * c.n_rg + row / kRowsPerWave;
  int64_t at = positions_before(d, r, lane);
  for (int k = 0; k < j; ++k)
    at += static_cast<int64_t>(stream_span(tile_chunks(
              request_tile(r, q_start, q_len, seq_len, c.bq, k), c.window, c.causal != 0))) *
          c.n_hg;
  const int32_t n = tile_chunks(request_tile(r, q_start, q_len, seq_len, c.bq, j), c.window,
                                c.causal != 0);
  int first, live;
  stream_splits(at + static_cast<int64_t>(hu / c.gu) * stream_span(n), n, per, first, live);
  return live;
}

// Splits of row (tok, head) on the op path: the count the attention kernel
// recorded in the row's last log2-LSE slot (a quiet NaN with the count as
// payload, attn_device.h), or all num_splits when the slot holds a real LSE.
__device__ __forceinline__ uint32_t marker_bits(const CombineParams& c, int64_t tok, int head) {
  return *reinterpret_cast<const uint32_t*>(
      c.ws_lse + static_cast<int64_t>(c.num_splits - 1) * c.s_wl_split + tok * c.s_wl_tok +
      static_cast<int64_t>(head) * c.s_wl_head);
}
__device__ __forceinline__ int splits_of_marker(const CombineParams& c, uint32_t bits) {
  const uint32_t n = bits & 0x003fffffu;
  return (bits & 0xffc00000u) == 0x7fc00000u && n >= 1 && n < static_cast<uint32_t>(c.num_splits)
             ? static_cast<int>(n)
             : c.num_splits;
}


// NC consecutive fp32 columns at p (4 NC-byte aligned).
template <int NC>
__device__ __forceinline__ void load_cols(const char* p, float (&x)[NC]) {
  if constexpr (NC == 4) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(p);
    x[0] = t[0]; x[1] = t[1]; x[2] = t[2]; x[3] = t[3];
  } else if constexpr (NC == 2) {
    const f32x2 t = *reinterpret_cast<const f32x2*>(p);
    x[0] = t[0]; x[1] = t[1];
  } else {
    x[0] = *reinterpret_cast<const float*>(p);
  }
}

// Merges splits of the 64-split blocks first, first + step, ... of row
// (tok, head): the maximum M of their log2-LSEs and, relative to it, this
// lane's NC numerator columns and the (wave-summed) denominator.
template <int NC, int kBlk = 64>
__device__ __forceinline__ void merge_blocks(const CombineParams& c, int64_t tok, int head, int S,
                                             int first, int step, int lane, float& M,
                                             float (&num)[NC], float& den) {
  constexpr int kB = kBatch<NC> < kBlk ? kBatch<NC> : kBlk;
  const char* lse_row = c.ws_lse + tok * c.s_wl_tok + static_cast<int64_t>(head) * c.s_wl_head;
  const char* o_row =
      c.ws_o + tok * c.s_wo_tok + static_cast<int64_t>(head) * c.s_wo_head + 4 * NC * lane;
  M = kNegInf;
  if (lane < kBlk) {
    for (int s = kBlk * first + lane; s < S; s += kBlk * step) {
      const float x = *reinterpret_cast<const float*>(lse_row + s * c.s_wl_split);
      M = x > M ? x : M;  // -inf and NaN never win
    }
  }
  M = wave_max(M);
#pragma unroll
  for (int i = 0; i < NC; ++i) num[i] = 0.0f;
  den = 0.0f;
  if (!(M > kNegInf)) return;
  float den_l = 0.0f;
  for (int s0 = kBlk * first; s0 < S; s0 += kBlk * step) {
    const int s = s0 + lane;
    const float x = lane < kBlk && s < S ? *reinterpret_cast<const float*>(lse_row + s * c.s_wl_split)
                                         : kNegInf;
    const float w_l = x > kNegInf ? __builtin_amdgcn_exp2f(x - M) : 0.0f;
    den_l += w_l;
    const int n = S - s0 < kBlk ? S - s0 : kBlk;
    for (int e0 = 0; e0 < n; e0 += kB) {
      float w[kB];
      float ov[kB][NC];
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int e = e0 + k;
        w[k] = e < n ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                      __builtin_bit_cast(int, w_l), e))
                     : 0.0f;
        if (w[k] > 0.0f) {
          load_cols<NC>(o_row + (s0 + e) * c.s_wo_split, ov[k]);
        } else {
#pragma unroll
          for (int i = 0; i < NC; ++i) ov[k][i] = 0.0f;
        }
      }
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        if (w[k] > 0.0f) {
#pragma unroll
          for (int i = 0; i < NC; ++i) num[i] = fmaf(w[k], ov[k][i], num[i]);
        }
      }
    }
  }
  den = wave_sum(den_l);
}

// Partial rows merge_one_block issues per batch: a load batch, at most a block.
template <int NC, int kBlk>
constexpr int kOneBatch = kBatch<NC> < kBlk ? kBatch<NC> : kBlk;

// The partial rows of splits kBlk first + k, k < kSpec (at most the first
// batch merge_one_block merges), loaded before the split count is known:
// every slot below num_splits is workspace memory, and a row whose split
// turns out to have no weight (past the count, or -inf) never enters an
// arithmetic operation. kSpec trades the round trip saved against the rows
// read for nothing: few for many rows with few live splits each, the whole
// batch for few rows with many.
template <int NC, int kBlk, int kSpec>
__device__ __forceinline__ void spec_rows(const CombineParams& c, int64_t tok, int head,
                                          int first, int lane, float (&ov)[kSpec][NC]) {
  static_assert(kSpec >= 1 && kSpec <= kOneBatch<NC, kBlk>, "speculative rows: the first batch");
  const char* o_row =
      c.ws_o + tok * c.s_wo_tok + static_cast<int64_t>(head) * c.s_wo_head + 4 * NC * lane;
#pragma unroll
  for (int k = 0; k < kSpec; ++k) {
    const int s = kBlk * first + k;
    if (s < c.num_splits) {
      load_cols<NC>(o_row + static_cast<int64_t>(s) * c.s_wo_split, ov[k]);
    } else {
#pragma unroll
      for (int i = 0; i < NC; ++i) ov[k][i] = 0.0f;
    }
  }
}

// Merge of block `first` alone (every split of the row lies in the wave's
// one block), with the block's log2-LSEs already loaded: x_spec is lane l's
// slot kBlk first + l, read before the split count S was known, so lanes at
// or past S drop it. Same arithmetic in the same order as merge_blocks, so
// the results are identical; the partial rows are issued kOB at a time.
template <int NC, int kBlk, int kSpec>
__device__ __forceinline__ void merge_one_block(const CombineParams& c, int64_t tok, int head,
                                                int S, int first, float x_spec,
                                                const float (&ov_spec)[kSpec][NC], int lane,
                                                float& M, float (&num)[NC], float& den) {
  constexpr int kOB = kOneBatch<NC, kBlk>;
  const char* o_row =
      c.ws_o + tok * c.s_wo_tok + static_cast<int64_t>(head) * c.s_wo_head + 4 * NC * lane;
  const int s0 = kBlk * first;
  const float x = lane < kBlk && s0 + lane < S ? x_spec : kNegInf;
  M = wave_max(x > kNegInf ? x : kNegInf);  // NaN never wins
#pragma unroll
  for (int i = 0; i < NC; ++i) num[i] = 0.0f;
  den = 0.0f;
  if (!(M > kNegInf)) return;
  const float w_l = x > kNegInf ? __builtin_amdgcn_exp2f(x - M) : 0.0f;
  const int n = S - s0 < kBlk ? S - s0 : kBlk;
  for (int e0 = 0; e0 < n; e0 += kOB) {
    float w[kOB];
    float ov[kOB][NC];
#pragma unroll
    for (int k = 0; k < kOB; ++k) {
      const int e = e0 + k;
      w[k] = e < n ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                    __builtin_bit_cast(int, w_l), e))
                   : 0.0f;
      if (e0 == 0 && k < kSpec) {  // loaded with the LSEs
#pragma unroll
        for (int i = 0; i < NC; ++i) ov[k][i] = ov_spec[k < kSpec ? k : 0][i];
      } else if (w[k] > 0.0f) {
        load_cols<NC>(o_row + (s0 + e) * c.s_wo_split, ov[k]);
      } else {
#pragma unroll
        for (int i = 0; i < NC; ++i) ov[k][i] = 0.0f;
      }
    }
#pragma unroll
    for (int k = 0; k < kOB; ++k) {
      if (w[k] > 0.0f) {
#pragma unroll
        for (int i = 0; i < NC; ++i) num[i] = fmaf(w[k], ov[k][i], num[i]);
      }
    }
  }
  den = wave_sum(w_l);
}

// Lane l's log2-LSE slot kBlk first + l of row (tok, head), or -inf past the
// launch's splits.
template <int kBlk>
__device__ __forceinline__ float lse_slot(const CombineParams& c, int64_t tok, int head, int first,
                                          int lane) {
  const int s = kBlk * first + lane;
  if (lane >= kBlk || s >= c.num_splits) return kNegInf;
  return *reinterpret_cast<const float*>(c.ws_lse + tok * c.s_wl_tok +
                                         static_cast<int64_t>(head) * c.s_wl_head +
                                         static_cast<int64_t>(s) * c.s_wl_split);
}

template <int NC>
__device__ __forceinline__ void write_row(const CombineParams& c, int64_t tok, int head, float M,
                                          const float (&num)[NC], float den, int lane) {
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  float r[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) r[i] = num[i] * inv;
  char* dst = c.out + tok * c.s_out_tok + static_cast<int64_t>(head) * c.s_out_head;
  if (c.out_dtype == PTH_ATTN_BF16) {
    if constexpr (NC == 4) {
      *reinterpret_cast<bf16x4*>(dst + 8 * lane) =
          __builtin_convertvector((f32x4){r[0], r[1], r[2], r[3]}, bf16x4);
    } else if constexpr (NC == 2) {
      *reinterpret_cast<bf16x2*>(dst + 4 * lane) =
          __builtin_convertvector((f32x2){r[0], r[1]}, bf16x2);
    } else {
      *reinterpret_cast<__bf16*>(dst + 2 * lane) = static_cast<__bf16>(r[0]);
    }
  } else if (c.out_dtype == PTH_ATTN_F16) {
    if constexpr (NC == 4) {
      *reinterpret_cast<f16x4*>(dst + 8 * lane) =
          (f16x4){static_cast<_Float16>(r[0]), static_cast<_Float16>(r[1]),
                  static_cast<_Float16>(r[2]), static_cast<_Float16>(r[3])};
    } else if constexpr (NC == 2) {
      *reinterpret_cast<f16x2*>(dst + 4 * lane) =
          (f16x2){static_cast<_Float16>(r[0]), static_cast<_Float16>(r[1])};
    } else {
      *reinterpret_cast<_Float16*>(dst + 2 * lane) = static_cast<_Float16>(r[0]);
    }
  } else {
    if constexpr (NC == 4) {
      *reinterpret_cast<f32x4*>(dst + 16 * lane) = (f32x4){r[0], r[1], r[2], r[3]};
    } else if constexpr (NC == 2) {
      *reinterpret_cast<f32x2*>(dst + 8 * lane) = (f32x2){r[0], r[1]};
    } else {
      *reinterpret_cast<float*>(dst + 4 * lane) = r[0];
    }
  }
  if (c.lse_out != nullptr && lane == 0) {
    float* lo = reinterpret_cast<float*>(reinterpret_cast<char*>(c.lse_out) + tok * c.s_lo_tok +
                                         static_cast<int64_t>(head) * c.s_lo_head);
    *lo = den > 0.0f ? (M + __builtin_amdgcn_logf(den)) * 0.69314718055994530942f : kNegInf;
  }
}

// One wave per (token, head) row, whatever its split count.
template <int D>
__global__ __launch_bounds__(256) void combine_splits(const CombineParams c) {
  constexpr int NC = D / 64;  // columns per lane
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  const int64_t tok = row / c.num_q_heads;
  const int head = static_cast<int>(row - tok * c.num_q_heads);
  if (tok >= c.num_tokens) return;
  // The marker, the padding bound, the first 64 LSEs and the first batch of
  // partial rows are loaded in one round; a row whose splits (the marker's
  // count) fit one 64-split block is then merged without another LSE round.
  const int bound = ld_ro(c.qsl, c.num_reqs);
  const uint32_t bits = marker_bits(c, tok, head);  // read on every path: the slot exists
  const float x_spec = lse_slot<64>(c, tok, head, 0, lane);
  constexpr int kSpec = 4;  // many rows, few live splits each
  float ov_spec[kSpec][NC];
  spec_rows<NC, 64, kSpec>(c, tok, head, 0, lane, ov_spec);
  // One round: the compiler would otherwise issue the marker load only after
  // the padding-bound test below (a second dependent round trip).
  asm volatile("" ::"s"(bits), "s"(bound) : "memory");
  if (tok >= bound) return;  // padding row
  const int S = c.seq_lens != nullptr ? splits_of_marker(c, bits) : c.num_splits;
  if (c.seq_lens != nullptr && S == 1) return;  // written to out by the attention kernel
  float M, den;
  float num[NC];
  if (S <= 64)
    merge_one_block<NC, 64, kSpec>(c, tok, head, S, 0, x_spec, ov_spec, lane, M, num, den);
  else
    merge_blocks<NC>(c, tok, head, S, 0, 1, lane, M, num, den);
  write_row<NC>(c, tok, head, M, num, den, lane);
}

// Few rows with more than 512 splits (shared_rows): a work-group of 16 waves
// per row; wave w merges the 16-split blocks w, w + 16, ... and wave 0 merges
// the 16 results in a fixed order. Beyond 512 the workspace is an upper bound
// and a row's live splits are often few (config 1: 32 of 2048), which
// 16-split blocks spread over more waves. (Up to 512 splits, combine_cols
// below.)
constexpr int kSharedWaves = 16;

template <int D, int kSharedBlock>
__global__ __launch_bounds__(kSharedWaves * 64) void combine_shared(const CombineParams c) {
  constexpr int NC = D / 64;
  __shared__ float part_m[kSharedWaves], part_den[kSharedWaves];
  __shared__ float part_num[kSharedWaves][NC][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = blockIdx.x;
  const int64_t tok = row / c.num_q_heads;
  const int head = static_cast<int>(row - tok * c.num_q_heads);
  if (tok >= c.num_tokens) return;  // uniform over the work-group
  // The padding bound, the marker, the wave's block of LSEs and its first
  // batch of partial rows are loaded in one round; when the row's splits (the
  // marker's count) fit one block per wave no further LSE round follows.
  const int bound = ld_ro(c.qsl, c.num_reqs);
  const uint32_t bits = marker_bits(c, tok, head);  // read on every path: the slot exists
  const float x_spec = lse_slot<kSharedBlock>(c, tok, head, wave, lane);
  constexpr int kSpec = kOneBatch<NC, kSharedBlock>;  // few rows, many splits each
  float ov_spec[kSpec][NC];
  spec_rows<NC, kSharedBlock, kSpec>(c, tok, head, wave, lane, ov_spec);
  // One round: the compiler would otherwise issue the marker load only after
  // the padding-bound test below (a second dependent round trip).
  asm volatile("" ::"s"(bits), "s"(bound) : "memory");
  if (tok >= bound) return;  // padding row, uniform over the work-group
  const int S = c.seq_lens != nullptr ? splits_of_marker(c, bits) : c.num_splits;
  if (c.seq_lens != nullptr && S == 1) return;  // written to out by the attention kernel
  if (S <= kSharedWaves * kSharedBlock && kSharedBlock * wave >= S) {
    // No live split in this wave's block: an empty result, without waiting
    // for the partial rows loaded speculatively (slots nobody wrote, often
    // the slowest loads of the round).
    if (lane == 0) {
      part_m[wave] = kNegInf;
      part_den[wave] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) part_num[wave][i][lane] = 0.0f;
    __syncthreads();
    return;
  }
  float M, den;
  float num[NC];
  if (S <= kSharedWaves * kSharedBlock)
    merge_one_block<NC, kSharedBlock, kSpec>(c, tok, head, S, wave, x_spec, ov_spec, lane, M,
                                             num, den);
  else
    merge_blocks<NC, kSharedBlock>(c, tok, head, S, wave, kSharedWaves, lane, M, num, den);
  if (lane == 0) {
    part_m[wave] = M;
    part_den[wave] = den;
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) part_num[wave][i][lane] = num[i];
  __syncthreads();
  if (wave != 0) return;
  // Every wave's result read at once (one LDS round trip), then merged in
  // wave order.
  float pm[kSharedWaves], pd[kSharedWaves], pn[kSharedWaves][NC];
#pragma unroll
  for (int w = 0; w < kSharedWaves; ++w) {
    pm[w] = part_m[w];
    pd[w] = part_den[w];
#pragma unroll
    for (int i = 0; i < NC; ++i) pn[w][i] = part_num[w][i][lane];
  }
  float Mg = kNegInf;
#pragma unroll
  for (int w = 0; w < kSharedWaves; ++w) Mg = pm[w] > Mg ? pm[w] : Mg;
  float ng[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) ng[i] = 0.0f;
  float dg = 0.0f;
  if (Mg > kNegInf) {
#pragma unroll
    for (int w = 0; w < kSharedWaves; ++w) {
      if (pm[w] > kNegInf) {
        const float a = __builtin_amdgcn_exp2f(pm[w] - Mg);
#pragma unroll
        for (int i = 0; i < NC; ++i) ng[i] = fmaf(a, pn[w][i], ng[i]);
        dg = fmaf(a, pd[w], dg);
      }
    }
  }
  write_row<NC>(c, tok, head, Mg, ng, dg, lane);
}

// Few rows with up to 16 kBlk splits each, split by columns as well: a
// work-group of 16 waves per (row, 32 columns), so a row's partials are read
// by D / 32 compute units instead of one (config 3's 32 rows then use 128
// compute units, the D = 256 decode's 12 rows 96). Wave w merges the splits
// of block w, two splits per load instruction (lanes 0-31 split 2k, lanes
// 32-63 split 2k + 1, one column each), the two halves are added, and wave 0
// merges the 16 waves in a fixed order. Loads are ordered by round as in
// combine_shared: the marker, the padding bound, the wave's LSEs and all its
// partial columns in one round.
constexpr int kColsPerPart = 32;

template <int D, int kBlk>
__global__ __launch_bounds__(kSharedWaves * 64) void combine_cols(const CombineParams c) {
  constexpr int kParts = D / kColsPerPart;
  constexpr int kLd = kBlk / 2;  // partial loads per lane
  __shared__ float part_m[kSharedWaves], part_den[kSharedWaves];
  __shared__ float part_num[kSharedWaves][kColsPerPart];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = blockIdx.x / kParts;
  const int part = static_cast<int>(blockIdx.x - row * kParts);
  const int64_t tok = row / c.num_q_heads;
  const int head = static_cast<int>(row - tok * c.num_q_heads);
  if (tok >= c.num_tokens) return;  // uniform over the work-group
  const int bound = ld_ro(c.qsl, c.num_reqs);
  const uint32_t bits = marker_bits(c, tok, head);  // read on every path: the slot exists
  const float x_spec = lse_slot<kBlk>(c, tok, head, wave, lane);
  const int half = lane >> 5;
  const int col = kColsPerPart * part + (lane & 31);
  const char* o_col =
      c.ws_o + tok * c.s_wo_tok + static_cast<int64_t>(head) * c.s_wo_head + 4 * col;
  const int s0 = kBlk * wave;
  float ov[kLd];
#pragma unroll
  for (int k = 0; k < kLd; ++k) {
    const int s = s0 + 2 * k + half;
    ov[k] = s < c.num_splits
                ? *reinterpret_cast<const float*>(o_col + static_cast<int64_t>(s) * c.s_wo_split)
                : 0.0f;
  }
  // One round: the compiler would otherwise issue the marker load only after
  // the padding-bound test below (a second dependent round trip).
  asm volatile("" ::"s"(bits), "s"(bound) : "memory");
  if (tok >= bound) return;  // padding row, uniform over the work-group
  const int S = c.seq_lens != nullptr ? splits_of_marker(c, bits) : c.num_splits;
  if (c.seq_lens != nullptr && S == 1) return;  // written to out by the attention kernel
  const float x = lane < kBlk && s0 + lane < S ? x_spec : kNegInf;
  const float M = wave_max(x > kNegInf ? x : kNegInf);  // NaN never wins
  float num = 0.0f, den = 0.0f;
  if (M > kNegInf) {
    const float w_l = x > kNegInf ? __builtin_amdgcn_exp2f(x - M) : 0.0f;
#pragma unroll
    for (int k = 0; k < kLd; ++k) {
      const float wa = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_l), 2 * k));
      const float wb = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_l), 2 * k + 1));
      const float w = half ? wb : wa;
      if (w > 0.0f) num = fmaf(w, ov[k], num);
    }
    den = wave_sum(w_l);
  }
  num += __shfl_xor(num, 32);  // the two halves of the column (commutative)
  if (lane == 0) {
    part_m[wave] = M;
    part_den[wave] = den;
  }
  if (lane < kColsPerPart) part_num[wave][lane] = num;
  __syncthreads();
  if (wave != 0 || lane >= kColsPerPart) return;
  // Every wave's result read at once (one LDS round trip), then merged in
  // wave order.
  float pm[kSharedWaves], pd[kSharedWaves], pn[kSharedWaves];
#pragma unroll
  for (int w = 0; w < kSharedWaves; ++w) {
    pm[w] = part_m[w];
    pd[w] = part_den[w];
    pn[w] = part_num[w][lane];
  }
  float Mg = kNegInf;
#pragma unroll
  for (int w = 0; w < kSharedWaves; ++w) Mg = pm[w] > Mg ? pm[w] : Mg;
  float ng = 0.0f, dg = 0.0f;
  if (Mg > kNegInf) {
#pragma unroll
    for (int w = 0; w < kSharedWaves; ++w) {
      if (pm[w] > kNegInf) {
        const float a = __builtin_amdgcn_exp2f(pm[w] - Mg);
        ng = fmaf(a, pn[w], ng);
        dg = fmaf(a, pd[w], dg);
      }
    }
  }
  const float r = dg > 0.0f ? ng * (1.0f / dg) : 0.0f;
  char* dst = c.out + tok * c.s_out_tok + static_cast<int64_t>(head) * c.s_out_head;
  if (c.out_dtype == PTH_ATTN_BF16)
    *reinterpret_cast<__bf16*>(dst + 2 * col) = static_cast<__bf16>(r);
  else if (c.out_dtype == PTH_ATTN_F16)
    *reinterpret_cast<_Float16*>(dst + 2 * col) = static_cast<_Float16>(r);
  else
    *reinterpret_cast<float*>(dst + 4 * col) = r;
  if (c.lse_out != nullptr && part == 0 && lane == 0) {
    float* lo = reinterpret_cast<float*>(reinterpret_cast<char*>(c.lse_out) + tok * c.s_lo_tok +
                                         static_cast<int64_t>(head) * c.s_lo_head);
    *lo = dg > 0.0f ? (Mg + __builtin_amdgcn_logf(dg)) * 0.69314718055994530942f : kNegInf;
  }
}

// -inf into the log2-LSE slot of every split s >= live of every query row
// (live: the splits the attention kernel wrote for the row), so that a
// combine over all num_splits splits ignores them, as the reference's launch
// contract requires of the split partials (reference attn_args.h:38-44). One
// wave per row; padding rows are not written.
__global__ __launch_bounds__(256) void fill_unused_splits(const CombineParams c) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  const int64_t tok = row / c.num_q_heads;
  const int head = static_cast<int>(row - tok * c.num_q_heads);
  if (tok >= c.num_tokens) return;
  const int r = request_of_token(c, tok, lane);
  if (r >= c.num_reqs) return;
  const int live = row_live_splits(c, r, tok, head, lane);
  char* lse_row = const_cast<char*>(c.ws_lse) + tok * c.s_wl_tok + static_cast<int64_t>(head) * c.s_wl_head;
  for (int s = live + lane; s < c.num_splits; s += 64)
    *reinterpret_cast<float*>(lse_row + s * c.s_wl_split) = kNegInf;
}

template <int D>
void launch_combine_d(const CombineParams& c, int64_t rows, hipStream_t stream) {
  const unsigned parts = static_cast<unsigned>(D / kColsPerPart);
  if (c.shared_rows && c.num_splits <= kSharedWaves * 16)
    hipLaunchKernelGGL((combine_cols<D, 16>), dim3(static_cast<unsigned>(rows) * parts),
                       dim3(kSharedWaves * 64), 0, stream, c);
  else if (c.shared_rows && c.num_splits <= kSharedWaves * 32)
    hipLaunchKernelGGL((combine_cols<D, 32>), dim3(static_cast<unsigned>(rows) * parts),
                       dim3(kSharedWaves * 64), 0, stream, c);
  else if (c.shared_rows)
    hipLaunchKernelGGL((combine_shared<D, 16>), dim3(static_cast<unsigned>(rows)),
                       dim3(kSharedWaves * 64), 0, stream, c);
  else
    hipLaunchKernelGGL(combine_splits<D>, dim3(static_cast<unsigned>((rows + kWaves - 1) / kWaves)),
                       dim3(kWaves * 64), 0, stream, c);
}

}  // namespace

hipError_t launch_fill_unused_splits(const CombineParams& c, hipStream_t stream) {
  const int64_t rows = static_cast<int64_t>(c.num_tokens) * c.num_q_heads;
  const unsigned blocks = static_cast<unsigned>((rows + kWaves - 1) / kWaves);
  hipLaunchKernelGGL(fill_unused_splits, dim3(blocks), dim3(kWaves * 64), 0, stream, c);
  return hipGetLastError();
}

hipError_t launch_combine_kernel(const CombineParams& c, hipStream_t stream) {
  const int64_t rows = static_cast<int64_t>(c.num_tokens) * c.num_q_heads;
  switch (c.head_size) {
    case 64: launch_combine_d<64>(c, rows, stream); break;
    case 256: launch_combine_d<256>(c, rows, stream); break;
    default: launch_combine_d<128>(c, rows, stream);
  }
  return hipGetLastError();
}

}  // namespace pa
