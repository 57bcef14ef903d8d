// attn_fwd.hip -- the gfx950 paged int8 attention kernel, D = 128.
//
// Work decomposition. A work unit is (request, row tile, split, KV head,
// 16-row group); a row tile holds up to bq query tokens of one request and
// its rows are (token, head-in-group) pairs, token-major (reference
// cache_geometry.cuh:319-334). The kernel is persistent: the grid is one
// wave64 per resident slot of the GPU (CUs x 8) and wave w runs units
// w, w + W, w + 2W, ... of a table that it derives on the device from
// query_start_loc and seq_lens (a prefix sum over requests, 64 requests per
// wave instruction), so the launch is graph-safe and no work-group is ever
// spent on an empty split. Each request uses as many splits as its length
// needs (at least 4 KV tiles each, at most the planner's S). The KV head is
// the fastest index of the table: the 4 waves of a work-group take 4 adjacent
// heads of one (row tile, split), whose cache cells are adjacent in memory,
// so the lines they share are fetched into L2 once.
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
// max is reduced over the 4 lanes of a row with two xor shuffles; the
// running sum stays per lane and is reduced once at the end.

#include "attn_internal.h"

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

__device__ __forceinline__ float xor_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float xor_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// The cache bytes of one 32-key chunk for one lane.
struct Chunk {
  u32x4 k[2][2];  // K: 32 bytes of key (16 sub + r) for sub = 0, 1
  u32x2 v[8];     // V: 8 bytes of key tv(e)
  float sc;       // one scale: see load_chunk
};

// Lane n of every 16-lane row, broadcast to the row (DPP row_newbcast).
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x),
                                                            0x150 + N, 0xf, 0xf, false));
}

__device__ __forceinline__ const char* at(const CacheStream& s, int64_t page,
                                          int32_t slot, int32_t head) {
  return s.base + page * s.s_block + static_cast<int64_t>(slot) * s.s_slot +
         static_cast<int64_t>(head) * s.s_head;
}

// One work unit: rows [16 rg, 16 rg + 16) of row tile t, KV head kvh, split
// s of the row tile's `live` splits.
template <bool kWindow, bool kPaged16, bool kF16Q>
__device__ __forceinline__ void run_unit(const AttnParams& p, const RowTile& t, int s,
                                         int live, int kvh, int rg, int lane) {
  const int G = p.group;
  const int rows = t.num_tok * G;
  const int row0 = rg * kRowsPerWave;
  if (row0 >= rows) return;

  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int row = row0 + r16;
  const bool vrow = row < rows;
  const int tok = static_cast<int>(p.g_div.div(static_cast<uint32_t>(vrow ? row : row0)));
  const int head = kvh * G + ((vrow ? row : row0) - tok * G);
  const int64_t qtok = static_cast<int64_t>(t.q_start) + t.tok_begin + tok;
  const int window = kWindow ? p.window : 0;
  const bool causal = kWindow ? (p.causal != 0) : true;
  const int lo = key_lo(t, t.tok_begin + tok, window);
  const int hi = key_hi(t, t.tok_begin + tok, window, causal);

  // Key bounds of the wave's real rows (uniform): first and last token.
  const int wrow_end = (row0 + kRowsPerWave < rows ? row0 + kRowsPerWave : rows);
  const int tok_first = static_cast<int>(p.g_div.div(row0));
  const int tok_last = static_cast<int>(p.g_div.div(wrow_end - 1));
  const int w_lo_min = key_lo(t, t.tok_begin + tok_first, window);
  const int w_lo_max = key_lo(t, t.tok_begin + tok_last, window);
  const int w_hi_min = key_hi(t, t.tok_begin + tok_first, window, causal);
  const int w_hi_max = key_hi(t, t.tok_begin + tok_last, window, causal);

  // Split of the row tile's KV tiles (the same for every wave of the tile).
  const int rbeg = kWindow ? range_begin(t, window) : 0;
  const int rend = range_end(t, window, causal);
  const int ft = first_kv_tile(rbeg);
  const int nt = kv_tile_count(rbeg, rend);
  const bool split_out = p.num_splits > 1;
  if (split_out && s == live - 1 && vrow) {
    // Splits [live, S) of this request hold no key of these rows: lse = -inf,
    // so that any combine over all S splits skips them.
    char* lse_row = reinterpret_cast<char*>(p.ws_lse) + qtok * p.s_wl_tok +
                    static_cast<int64_t>(head) * p.s_wl_head;
    for (int s2 = live + g; s2 < p.num_splits; s2 += 4)
      *reinterpret_cast<float*>(lse_row + s2 * p.s_wl_split) = kNegInf;
  }
  int tb, te;
  split_range(s, live, nt, tb, te);
  // Keys this wave reads: its split's tiles, clipped to its rows' keys.
  const int c_split_lo = (ft + tb) * kTileTokens;
  const int c_split_hi = (ft + te) * kTileTokens;
  const int ld_lo = c_split_lo > w_lo_min ? c_split_lo : w_lo_min;
  const int ld_hi = c_split_hi < w_hi_max + 1 ? c_split_hi : w_hi_max + 1;
  const int c_begin = ld_lo & ~(kChunkTokens - 1);

  // Q^T as the B operand: qb[j] holds Q[row][32 g + 8 j .. + 8].
  bf16x8 qb[4], qb_lo[4];
  {
    const char* qrow = p.q + qtok * p.s_q_tok + static_cast<int64_t>(head) * p.s_q_head;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 raw = vrow ? *reinterpret_cast<const u32x4*>(qrow + 2 * (32 * g + 8 * j))
                       : (u32x4){0u, 0u, 0u, 0u};
      if constexpr (kF16Q) {
        // fp16 q = hi + lo with hi = bf16(q), lo = bf16(q - hi): exact, because
        // an fp16 significand has 11 bits and each bf16 holds 8.
        const f16x8 h = __builtin_bit_cast(f16x8, raw);
        bf16x8 a, b;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = static_cast<float>(h[e]);
          const __bf16 fh = static_cast<__bf16>(f);
          a[e] = fh;
          b[e] = static_cast<__bf16>(f - static_cast<float>(fh));
        }
        qb[j] = a;
        qb_lo[j] = b;
      } else {
        qb[j] = __builtin_bit_cast(bf16x8, raw);
      }
    }
  }

  const int req = t.req;
  const int32_t* bt_row = p.block_table + static_cast<int64_t>(req) * p.bt_stride;
  const int BS = static_cast<int>(p.bs_div.d);

  // Lane (r, g) also loads ONE scale: k_scale of key tv(r) for r < 8, v_scale
  // of key tv(r - 8) for r >= 8; a row broadcast hands them to the row.
  const int sc_e = r16 & 7;
  const CacheStream& sc_stream = r16 < 8 ? p.ks : p.vs;

  auto load_chunk = [&](int c, Chunk& ch) {
    if constexpr (kPaged16) {
      // BS % 16 == 0: the 16 keys of each half-chunk share one page (uniform).
      int64_t page[2];
      int slot0[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int c16 = c + 16 * sub;
        page[sub] = 0;
        slot0[sub] = 0;
        if (c16 < ld_hi && c16 + 16 > ld_lo) {
          const int blk = static_cast<int>(p.bs_div.div(c16));
          slot0[sub] = c16 - blk * BS;
          page[sub] = bt_row[blk];
        }
        const int tk = c16 + r16;
        const bool ok = tk >= ld_lo && tk < ld_hi;
        const char* kp = at(p.k, page[sub], slot0[sub] + r16, kvh) + 32 * g;
        ch.k[sub][0] = ok ? (u32x4)(*reinterpret_cast<const u32x4_a4*>(kp)) : (u32x4){0u, 0u, 0u, 0u};
        ch.k[sub][1] = ok ? (u32x4)(*reinterpret_cast<const u32x4_a4*>(kp + 16)) : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tv = c16 + 4 * g + i;
          const bool okv = tv >= ld_lo && tv < ld_hi;
          const char* vp = at(p.v, page[sub], slot0[sub] + 4 * g + i, kvh) + 8 * r16;
          ch.v[4 * sub + i] = okv ? (u32x2)(*reinterpret_cast<const u32x2_a4*>(vp)) : (u32x2){0u, 0u};
        }
      }
      const int sub_e = sc_e >> 2;
      const int ts = c + 16 * sub_e + 4 * g + (sc_e & 3);
      const bool oks = ts >= ld_lo && ts < ld_hi;
      const int64_t pg = sub_e ? page[1] : page[0];
      const int sl = (sub_e ? slot0[1] : slot0[0]) + 4 * g + (sc_e & 3);
      ch.sc = oks ? *reinterpret_cast<const float*>(at(sc_stream, pg, sl, kvh)) : 0.0f;
    } else {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int c16 = c + 16 * sub;
        const int tk = c16 + r16;
        u32x4 k0 = {0u, 0u, 0u, 0u}, k1 = {0u, 0u, 0u, 0u};
        if (tk >= ld_lo && tk < ld_hi) {
          const int blk = static_cast<int>(p.bs_div.div(tk));
          const char* kp = at(p.k, bt_row[blk], tk - blk * BS, kvh) + 32 * g;
          k0 = *reinterpret_cast<const u32x4_a4*>(kp);
          k1 = *reinterpret_cast<const u32x4_a4*>(kp + 16);
        }
        ch.k[sub][0] = k0;
        ch.k[sub][1] = k1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tv = c16 + 4 * g + i;
          u32x2 vv = {0u, 0u};
          if (tv >= ld_lo && tv < ld_hi) {
            const int blk = static_cast<int>(p.bs_div.div(tv));
            vv = *reinterpret_cast<const u32x2_a4*>(at(p.v, bt_row[blk], tv - blk * BS, kvh) + 8 * r16);
          }
          ch.v[4 * sub + i] = vv;
        }
      }
      const int ts = c + 16 * (sc_e >> 2) + 4 * g + (sc_e & 3);
      float scv = 0.0f;
      if (ts >= ld_lo && ts < ld_hi) {
        const int blk = static_cast<int>(p.bs_div.div(ts));
        scv = *reinterpret_cast<const float*>(at(sc_stream, bt_row[blk], ts - blk * BS, kvh));
      }
      ch.sc = scv;
    }
  };

  f32x4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m = kNegInf;
  float l = 0.0f;
  const float scale_log2 = p.scale_log2;

  auto compute_chunk = [&](int c, const Chunk& ch) {
    const float ks[8] = {row_bcast<0>(ch.sc), row_bcast<1>(ch.sc), row_bcast<2>(ch.sc),
                         row_bcast<3>(ch.sc), row_bcast<4>(ch.sc), row_bcast<5>(ch.sc),
                         row_bcast<6>(ch.sc), row_bcast<7>(ch.sc)};
    const float vs[8] = {row_bcast<8>(ch.sc),  row_bcast<9>(ch.sc),  row_bcast<10>(ch.sc),
                         row_bcast<11>(ch.sc), row_bcast<12>(ch.sc), row_bcast<13>(ch.sc),
                         row_bcast<14>(ch.sc), row_bcast<15>(ch.sc)};
    float sc[8];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4& w = ch.k[sub][j >> 1];
        const bf16x8 a = (j & 1) ? i8x8_to_bf16(w[2], w[3]) : i8x8_to_bf16(w[0], w[1]);
        acc = mfma(a, qb[j], acc);
        if constexpr (kF16Q) acc = mfma(a, qb_lo[j], acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * sub + i] = acc[i] * (ks[4 * sub + i] * scale_log2);
    }
    const bool need_mask = c < w_lo_max || c + kChunkTokens - 1 > w_hi_min;
    if (need_mask) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tv = c + 16 * (e >> 2) + 4 * g + (e & 3);
        if (tv < lo || tv > hi) sc[e] = kNegInf;
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sc[e]);
    mx = xor_max(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == kNegInf ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    float pv[8];
    float lsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pe = __builtin_amdgcn_exp2f(sc[e] - m_use);
      lsum += pe;
      pv[e] = pe * vs[e];
    }
    l = l * alpha + lsum;
    m = m_new;
    // P = hi + lo in bf16 (16 significant bits together): a single bf16 P
    // would carry a 2^-9 relative error straight into the output whenever the
    // softmax is peaked (short contexts, early causal rows).
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
    for (int j = 0; j < 8; ++j) {
      o[j] *= alpha;
      const bf16x8 vcol = column_to_bf16(ch.v, j);
      o[j] = mfma(vcol, p_hi, o[j]);
      o[j] = mfma(vcol, p_lo, o[j]);
    }
  };

  // Two-buffer pipeline: the loads of chunk c + 32 are in flight while chunk
  // c is computed.
  if (c_begin < ld_hi) {
    Chunk ca, cb;
    int c = c_begin;
    load_chunk(c, ca);
    while (true) {
      if (c + kChunkTokens < ld_hi) load_chunk(c + kChunkTokens, cb);
      compute_chunk(c, ca);
      c += kChunkTokens;
      if (c >= ld_hi) break;
      if (c + kChunkTokens < ld_hi) load_chunk(c + kChunkTokens, ca);
      compute_chunk(c, cb);
      c += kChunkTokens;
      if (c >= ld_hi) break;
    }
  }

  const float l_tot = xor_sum(l);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (!vrow) return;
  float res[32];  // res[8 i + j] = column 32 g + 8 i + j
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) res[8 * i + j] = o[j][i] * inv;
  const float lse2 = l_tot > 0.0f ? m + __builtin_amdgcn_logf(l_tot) : kNegInf;

  if (split_out) {
    char* dst = reinterpret_cast<char*>(p.ws_o) + s * p.s_wo_split + qtok * p.s_wo_tok +
                static_cast<int64_t>(head) * p.s_wo_head + 4 * 32 * g;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      *reinterpret_cast<f32x4*>(dst + 16 * k) =
          (f32x4){res[4 * k], res[4 * k + 1], res[4 * k + 2], res[4 * k + 3]};
    if (g == 0) {
      float* lse = reinterpret_cast<float*>(reinterpret_cast<char*>(p.ws_lse) + s * p.s_wl_split +
                                            qtok * p.s_wl_tok +
                                            static_cast<int64_t>(head) * p.s_wl_head);
      *lse = lse2;
    }
    return;
  }
  char* dst = p.out + qtok * p.s_out_tok + static_cast<int64_t>(head) * p.s_out_head;
  if (p.out_dtype == PTH_ATTN_BF16) {
    dst += 2 * 32 * g;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf16x2 pr = pack_bf16(res[8 * k + e], res[8 * k + e + 1]);
        v[e] = pr[0];
        v[e + 1] = pr[1];
      }
      *reinterpret_cast<bf16x8*>(dst + 16 * k) = v;
    }
  } else if (p.out_dtype == PTH_ATTN_F16) {
    dst += 2 * 32 * g;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = static_cast<_Float16>(res[8 * k + e]);
      *reinterpret_cast<f16x8*>(dst + 16 * k) = v;
    }
  } else {
    dst += 4 * 32 * g;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      *reinterpret_cast<f32x4*>(dst + 16 * k) =
          (f32x4){res[4 * k], res[4 * k + 1], res[4 * k + 2], res[4 * k + 3]};
  }
  if (p.lse_out != nullptr && g == 0) {
    float* lo_ptr = reinterpret_cast<float*>(reinterpret_cast<char*>(p.lse_out) +
                                             qtok * p.s_lo_tok +
                                             static_cast<int64_t>(head) * p.s_lo_head);
    *lo_ptr = lse2 * 0.69314718055994530942f;
  }
}


// The persistent worker loop (see the header comment for the unit table).
template <bool kWindow, bool kPaged16, bool kF16Q>
__global__ __launch_bounds__(256, 2) void attn_fwd_d128(const AttnParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int worker = blockIdx.x * kWaves + wave;
  const int num_workers = gridDim.x * kWaves;
  const int R = p.num_reqs;
  const int n_hu = p.n_hu;
  const int bq = p.bq;
  const int window = kWindow ? p.window : 0;
  const bool causal = kWindow ? (p.causal != 0) : true;

  // The current 64-request chunk of the unit table: lane j describes request
  // chunk_r0 + j; incl is the inclusive prefix of units within the chunk.
  int chunk_r0 = -64;
  int chunk_u0 = 0, chunk_u1 = 0;
  int incl = 0;
  for (int u = worker;; u += num_workers) {
    bool done = false;
    while (u >= chunk_u1) {
      chunk_r0 += 64;
      chunk_u0 = chunk_u1;
      if (chunk_r0 >= R) {
        done = true;
        break;
      }
      const int r = chunk_r0 + lane;
      int units = 0;
      if (r < R) {
        const int ql = p.qsl[r + 1] - p.qsl[r];
        units = request_row_tiles(ql, bq) *
                request_splits(ql, p.seq_lens[r], bq, window, causal, p.num_splits) * n_hu;
      }
      incl = units;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
      }
      chunk_u1 = chunk_u0 + __builtin_amdgcn_readlane(incl, 63);
    }
    if (done) break;
    const int local = u - chunk_u0;
    const int j = static_cast<int>(__popcll(__ballot(incl <= local)));
    const int excl = j > 0 ? __builtin_amdgcn_readlane(incl, j - 1) : 0;
    const int u_loc = local - excl;
    const int req = chunk_r0 + j;
    const int q_start = p.qsl[req];
    const int q_len = p.qsl[req + 1] - q_start;
    const int seq_len = p.seq_lens[req];
    const int live = request_splits(q_len, seq_len, bq, window, causal, p.num_splits);
    const int hu = u_loc % n_hu;
    const int t2 = u_loc / n_hu;
    const int s = t2 % live;
    const int rt = t2 / live;
    const RowTile t = request_tile(req, q_start, q_len, seq_len, bq, rt);
    const int kvh = static_cast<int>(p.rg_div.div(hu));
    const int rg = hu - kvh * static_cast<int>(p.rg_div.d);
    run_unit<kWindow, kPaged16, kF16Q>(p, t, s, live, kvh, rg, lane);
  }
}

template <bool W, bool P, bool F>
hipError_t launch_one(const AttnParams& p, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_d128<W, P, F>), grid, dim3(kWaves * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_kernel(const AttnParams& p, dim3 grid, bool windowed,
                             bool paged16, bool q_f16, hipStream_t stream) {
  if (windowed) {
    if (paged16) return q_f16 ? launch_one<true, true, true>(p, grid, stream)
                              : launch_one<true, true, false>(p, grid, stream);
    return q_f16 ? launch_one<true, false, true>(p, grid, stream)
                 : launch_one<true, false, false>(p, grid, stream);
  }
  if (paged16) return q_f16 ? launch_one<false, true, true>(p, grid, stream)
                            : launch_one<false, true, false>(p, grid, stream);
  return q_f16 ? launch_one<false, false, true>(p, grid, stream)
               : launch_one<false, false, false>(p, grid, stream);
}

}  // namespace pa
