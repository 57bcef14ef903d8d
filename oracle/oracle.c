/*
 * oracle.c -- CPU restatement of the reference's answer for paged int8
 * attention. TEST INFRASTRUCTURE ONLY: imported by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
 * Never linked into, called by or shipped with the product path.
 *
 * Functions (each follows the reference file:line named in its comment):
 *  - oracle_quantize_rows: vLLM's int8 per-token-head writer as mirrored by
 *    python/pth_testing/reference.py:76-103 (quantize_rows), fp32 step for
 *    step: scale = max(absmax / 127, 1e-6); q = x * (1 / scale); +-0.5 away
 *    from zero; clamp [-128, 127]; truncate. Built with -ffp-contract=off so
 *    no step is fused.
 *  - oracle_attention: reference.py:596-671 (ref_attention) over the paged
 *    views as reference.py:241-258 (Int8Cache.dense) gathers them: fp64
 *    softmax attention of the dequantised cache (k_scale * k_int exactly),
 *    bottom-right causal / sliding window / non-causal per
 *    reference.py:553-593 (visible_mask), natural-log LSE; rows of tokens
 *    >= qsl[R] are not written. It takes the library's own PthAttnArgs with
 *    HOST pointers, so it reads the cache through exactly the same byte
 *    strides, block table and lengths as the kernel.
 *  - oracle_combine: combine_kernel.cuh:255-300 (combine_row) in fp64: M over
 *    live splits, w = 2^(lse - M), -inf splits skipped before o is read,
 *    fixed order s = 0..S-1.
 *
 * Parity of each is pinned in tests/test_oracle.py (known-answer vectors of
 * the reference's tests, the reference's own compiled CPU path
 * oracle/_ref/libpth_ref_host.so, closed forms and brute force).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "pth_attn.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- writer */
void oracle_quantize_rows(const float* x, int64_t rows, int32_t D, int8_t* q,
                          float* scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * D;
    float amax = 0.0f;
    for (int32_t d = 0; d < D; ++d) {
      const float a = fabsf(xr[d]);
      if (a > amax) amax = a;
    }
    float s = amax / 127.0f;
    if (!(s >= 1e-6f)) s = 1e-6f;
    const float inv = 1.0f / s;
    scale[r] = s;
    for (int32_t d = 0; d < D; ++d) {
      float v = xr[d] * inv;
      v = v >= 0.0f ? v + 0.5f : v - 0.5f;
      if (v < -128.0f) v = -128.0f;
      if (v > 127.0f) v = 127.0f;
      q[r * D + d] = (int8_t)v; /* C conversion truncates toward zero */
    }
  }
}

/* ------------------------------------------------------------- helpers */
static double load_q(const PthAttnArgs* a, int64_t tok, int32_t head, int32_t d) {
  const char* p = (const char*)a->q + tok * a->q_stride_token +
                  (int64_t)head * a->q_stride_head + 2 * (int64_t)d;
  uint16_t h;
  memcpy(&h, p, 2);
  if (a->q_dtype == PTH_ATTN_BF16) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
  }
  /* IEEE binary16 -> double */
  const int sign = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  double v;
  if (e == 0) v = ldexp((double)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexp((double)(m | 0x400), e - 25);
  return sign ? -v : v;
}

static const char* cell(const PthAttnStream* s, int64_t page, int64_t slot, int32_t head) {
  return (const char*)s->data + page * s->stride_block + slot * s->stride_slot +
         (int64_t)head * s->stride_head;
}

/* Visible key range of query token i of a request (reference.py:574-593). */
static void visible(int32_t L, int32_t q_len, int32_t i, int32_t window, int32_t causal,
                    int32_t* lo, int32_t* hi) {
  const int32_t p = L - q_len + i;
  *lo = window > 0 ? (p - window + 1 > 0 ? p - window + 1 : 0) : 0;
  if (causal) *hi = p;
  else if (window > 0) *hi = (p + window - 1 < L - 1) ? p + window - 1 : L - 1;
  else *hi = L - 1;
}

/* --------------------------------------------------------- attention */
/* out: fp64 [T, Hq, D] dense; lse: fp64 [T, Hq] natural log; valid: [T].
 * Rows of tokens that belong to no request are left as given. Returns 0, or
 * -1 on an inconsistent request (q_len > seq_len). `threads` <= 0 uses the
 * OpenMP default. Only rows with token in [row_begin, row_end) are computed
 * (row_end <= 0 means all), so a caller can time or check a sample. */
int oracle_attention(const PthAttnArgs* a, double* out, double* lse, uint8_t* valid,
                     int32_t threads, int64_t row_begin, int64_t row_end) {
  const int32_t T = a->num_tokens, Hq = a->num_q_heads, D = a->head_size;
  const int32_t Hkv = a->num_kv_heads, G = Hq / Hkv, R = a->num_reqs;
  const int32_t* qsl = a->query_start_loc;
  for (int32_t r = 0; r < R; ++r)
    if (qsl[r + 1] - qsl[r] > a->seq_lens[r]) return -1;
  const int64_t tb = row_begin > 0 ? row_begin : 0;
  const int64_t te = (row_end > 0 && row_end < T) ? row_end : T;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
  const int64_t n_rows = (te - tb) * Hq;
#pragma omp parallel
  {
    double qv[256], acc[256];
    double* sc = NULL;
    int32_t sc_cap = 0;
#pragma omp for schedule(dynamic, 4)
    for (int64_t idx = 0; idx < n_rows; ++idx) {
      const int64_t tok = tb + idx / Hq;
      const int32_t head = (int32_t)(idx % Hq);
      int32_t r = -1;
      for (int32_t k = 0; k < R; ++k)
        if (tok >= qsl[k] && tok < qsl[k + 1]) { r = k; break; }
      if (r < 0) continue;
      if (head == 0) valid[tok] = 1;
      const int32_t L = a->seq_lens[r], q_len = qsl[r + 1] - qsl[r];
      const int32_t i = (int32_t)(tok - qsl[r]);
      int32_t lo, hi;
      visible(L, q_len, i, a->window, a->causal, &lo, &hi);
      const int32_t kvh = head / G;
      const int32_t n = hi - lo + 1;
      if (n > sc_cap) {
        free(sc);
        sc_cap = n + 1024;
        sc = (double*)malloc(sizeof(double) * (size_t)sc_cap);
      }
      for (int32_t d = 0; d < D; ++d) qv[d] = load_q(a, tok, head, d);
      const int32_t* bt = a->block_table + (int64_t)r * a->block_table_row_stride;
      double m = -INFINITY;
      for (int32_t j = lo; j <= hi; ++j) {
        const int64_t page = bt[j / a->block_size];
        const int64_t slot = j % a->block_size;
        const int8_t* kr = (const int8_t*)cell(&a->k_cache, page, slot, kvh);
        float ksf;
        memcpy(&ksf, cell(&a->k_scale, page, slot, kvh), 4);
        const double ks = ksf;
        double dot = 0.0;
        for (int32_t d = 0; d < D; ++d) dot += qv[d] * (ks * (double)kr[d]);
        const double s = dot * (double)a->softmax_scale;
        sc[j - lo] = s;
        if (s > m) m = s;
      }
      for (int32_t d = 0; d < D; ++d) acc[d] = 0.0;
      double den = 0.0;
      for (int32_t j = lo; j <= hi; ++j) {
        const double pj = exp(sc[j - lo] - m);
        den += pj;
        const int64_t page = bt[j / a->block_size];
        const int64_t slot = j % a->block_size;
        const int8_t* vr = (const int8_t*)cell(&a->v_cache, page, slot, kvh);
        float vsf;
        memcpy(&vsf, cell(&a->v_scale, page, slot, kvh), 4);
        const double w = pj * (double)vsf;
        for (int32_t d = 0; d < D; ++d) acc[d] += w * (double)vr[d];
      }
      double* o = out + (tok * Hq + head) * (int64_t)D;
      for (int32_t d = 0; d < D; ++d) o[d] = acc[d] / den;
      lse[tok * Hq + head] = m + log(den);
    }
    free(sc);
  }
  return 0;
}

/* ----------------------------------------------------------- combine */
/* ws_o: fp32 [S, T, Hq, D] dense, ws_lse: fp32 [S, T, Hq] dense (log2
 * units), out: fp64 [T, Hq, D], lse_nat: fp64 [T, Hq] natural log. */
void oracle_combine(const float* ws_o, const float* ws_lse, int32_t S, int32_t T,
                    int32_t Hq, int32_t D, double* out, double* lse_nat) {
  for (int64_t row = 0; row < (int64_t)T * Hq; ++row) {
    double M = -INFINITY;
    for (int32_t s = 0; s < S; ++s) {
      const double x = ws_lse[(int64_t)s * T * Hq + row];
      if (x > M) M = x;
    }
    double* o = out + row * D;
    for (int32_t d = 0; d < D; ++d) o[d] = 0.0;
    if (!(M > -INFINITY)) {
      lse_nat[row] = -INFINITY;
      continue;
    }
    double den = 0.0;
    for (int32_t s = 0; s < S; ++s) {
      const double x = ws_lse[(int64_t)s * T * Hq + row];
      if (!(x > -INFINITY)) continue;
      const double w = exp2(x - M);
      den += w;
      const float* os = ws_o + ((int64_t)s * T * Hq + row) * D;
      for (int32_t d = 0; d < D; ++d) o[d] += w * (double)os[d];
    }
    for (int32_t d = 0; d < D; ++d) o[d] /= den;
    lse_nat[row] = (M + log2(den)) * log(2.0);
  }
}
