// attn_combine.hip -- merge of the split-KV partials (flash-decoding
// combine) for D = 128.
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
// One wave64 per (token, head) row; lane l owns columns 2 l and 2 l + 1, so a
// split's row is one coalesced 512-byte read. Lane s loads lse_s (64 splits
// per instruction); the weights are broadcast with readlane and the o loads
// of 8 splits are issued before their fused multiply-adds. When the launcher
// passes the request lengths, only the splits the attention kernel used for
// the row's request are read (the others hold -inf by construction).

#include "attn_internal.h"

namespace pa {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_inff();
constexpr int kBatch = 8;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) x = fmaxf(x, __shfl_xor(x, d));
  return x;
}
// Butterfly sum: every lane adds the same pairs (commutatively), so all lanes
// hold the same, order-fixed total.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) x += __shfl_xor(x, d);
  return x;
}

__global__ __launch_bounds__(256) void combine_d128(const CombineParams c) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  const int64_t tok = row / c.num_q_heads;
  const int head = static_cast<int>(row - tok * c.num_q_heads);
  if (tok >= c.num_tokens) return;

  // Request of the token: the number of requests that end at or before it.
  int r = 0;
  for (int r0 = 0; r0 < c.num_reqs; r0 += 64) {
    const int k = r0 + lane;
    const bool before = k < c.num_reqs && c.qsl[k + 1] <= tok;
    const int n = static_cast<int>(__popcll(__ballot(before)));
    r += n;
    if (n < 64) break;
  }
  if (r >= c.num_reqs) return;  // a padding row beyond qsl[R]
  int S = c.num_splits;
  if (c.seq_lens != nullptr) {
    const int q_start = c.qsl[r];
    S = request_splits(c.qsl[r + 1] - q_start, c.seq_lens[r], c.bq, c.window,
                       c.causal != 0, c.num_splits);
  }

  const char* lse_row = c.ws_lse + tok * c.s_wl_tok + static_cast<int64_t>(head) * c.s_wl_head;
  const char* o_row = c.ws_o + tok * c.s_wo_tok + static_cast<int64_t>(head) * c.s_wo_head + 8 * lane;

  float M = kNegInf;
  for (int s = lane; s < S; s += 64) {
    const float x = *reinterpret_cast<const float*>(lse_row + s * c.s_wl_split);
    M = x > M ? x : M;  // -inf and NaN never win
  }
  M = wave_max(M);
  f32x2 num = {0.0f, 0.0f};
  float den = 0.0f;
  if (M > kNegInf) {
    float den_l = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 64) {
      const int s = s0 + lane;
      const float x = s < S ? *reinterpret_cast<const float*>(lse_row + s * c.s_wl_split) : kNegInf;
      const float w_l = x > kNegInf ? __builtin_amdgcn_exp2f(x - M) : 0.0f;
      den_l += w_l;
      const int n = S - s0 < 64 ? S - s0 : 64;
      for (int e0 = 0; e0 < n; e0 += kBatch) {
        float w[kBatch];
        f32x2 ov[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int e = e0 + k;
          w[k] = e < n ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                        __builtin_bit_cast(int, w_l), e))
                       : 0.0f;
          ov[k] = w[k] > 0.0f ? *reinterpret_cast<const f32x2*>(o_row + (s0 + e) * c.s_wo_split)
                              : (f32x2){0.0f, 0.0f};
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          if (w[k] > 0.0f) {
            num[0] = fmaf(w[k], ov[k][0], num[0]);
            num[1] = fmaf(w[k], ov[k][1], num[1]);
          }
        }
      }
    }
    den = wave_sum(den_l);
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  const float r0 = num[0] * inv, r1 = num[1] * inv;
  char* dst = c.out + tok * c.s_out_tok + static_cast<int64_t>(head) * c.s_out_head;
  if (c.out_dtype == PTH_ATTN_BF16) {
    *reinterpret_cast<bf16x2*>(dst + 4 * lane) = __builtin_convertvector((f32x2){r0, r1}, bf16x2);
  } else if (c.out_dtype == PTH_ATTN_F16) {
    *reinterpret_cast<f16x2*>(dst + 4 * lane) = (f16x2){static_cast<_Float16>(r0), static_cast<_Float16>(r1)};
  } else {
    *reinterpret_cast<f32x2*>(dst + 8 * lane) = (f32x2){r0, r1};
  }
  if (c.lse_out != nullptr && lane == 0) {
    float* lo = reinterpret_cast<float*>(reinterpret_cast<char*>(c.lse_out) + tok * c.s_lo_tok +
                                         static_cast<int64_t>(head) * c.s_lo_head);
    *lo = den > 0.0f ? (M + __builtin_amdgcn_logf(den)) * 0.69314718055994530942f : kNegInf;
  }
}

}  // namespace

hipError_t launch_combine_kernel(const CombineParams& c, hipStream_t stream) {
  const int64_t rows = static_cast<int64_t>(c.num_tokens) * c.num_q_heads;
  const unsigned blocks = static_cast<unsigned>((rows + kWaves - 1) / kWaves);
  hipLaunchKernelGGL(combine_d128, dim3(blocks), dim3(kWaves * 64), 0, stream, c);
  return hipGetLastError();
}

}  // namespace pa
