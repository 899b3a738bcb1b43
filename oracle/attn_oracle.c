/*
 * attn_oracle.c — CPU oracle for the FlashAttention-2 forward.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline — never as the product path.  The product
 * (flash-attention_amd/) does not link, import or call anything here.
 *
 * Functions and the reference code they restate (paths in the reference repo):
 *
 *  oracle_attn_rows_f64 / oracle_attn_f64
 *      Exact attention in double precision on the (already fp16/bf16-quantised)
 *      inputs: two passes per query row (max, then sum of exp), natural-log
 *      LSE.  Restates the math of cpu_reference_attention
 *      (benchmark/cpp/correctness_v6.cu:23-72: S = scale * q.k, causal j > i
 *      excluded at :51-53, softmax-weighted sum of V) and of the torch
 *      reference pytorch_attention
 *      (benchmark/python/tests/test_pybind_correctness.py:23-27).  The LSE is
 *      new (the reference has none): LSE_i = ln sum_j exp(scale * q_i.k_j).
 *      `mutation` != 0 plants a known mistake (for the tests that prove the
 *      pinning checks can see such mistakes); 0 is the oracle proper.
 *
 *  oracle_ref_online_f32
 *      The reference CPU path itself, restated: fp32 single-pass online
 *      softmax with expf exactly as correctness_v6.cu:23-72 (m/l/acc update
 *      per key).  Used as the CPU baseline of bench.py ("port") and checked
 *      against oracle_attn_f64.
 *
 *  oracle_kernel_numerics
 *      Emulation of the reference GPU kernel's arithmetic with the correct
 *      K^T (see below): fp32 scores, key tiles of block_n, running max of raw
 *      scores, p = exp2(s*c - m*c) with c = scale*log2(e)
 *      (src/softmax/online_softmax.cuh:13-19, src/config/config.cuh:84),
 *      O and l rescaled by exp2((m_old - m_new)*c) (online_softmax.cuh:89-117),
 *      l summed from unrounded fp32 p (:135-152), P rounded to fp16/bf16
 *      with round-to-nearest-even before the PV product
 *      (src/forward/forward_v6_mma.cuh:19-38), fp32 accumulate, O normalised
 *      in fp32 and rounded to the output type (forward_v6_mma.cuh:206-234).
 *      Its error against the fp64 oracle is the "reference kernel's own
 *      error" that the GPU result must stay within 2x of.  The reference
 *      kernel's K fragment mapping reads K transposed within 16x8 blocks by
 *      static reading; the emulator deliberately uses the mathematically
 *      correct Q.K^T, since the oracle is the mathematics.
 *
 *  oracle_kernel_numerics_rows
 *      The same emulation for selected (head, row) pairs only, so the 2x bar
 *      can be checked on sampled rows of the full-size configs.
 *
 *  oracle_round_f16 / oracle_round_bf16
 *      float -> IEEE binary16 / bfloat16 with round-to-nearest-even (the
 *      __float2half_rn / __float22half2_rn rounding the reference uses), plus
 *      the quantised value back in float.
 *
 * Tensor layout everywhere: contiguous [B, H, N, D] fp32 (holding the
 * quantised values), O in the same layout, LSE [B, H, N].
 */
#include "attn_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* rounding                                                                 */
/* ------------------------------------------------------------------------ */

static uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal half */
    /* value / 2^-24, rounded to nearest even integer; exact scaling by 2^24 */
    const float scaled = fabsf(f) * 16777216.0f;
    const uint32_t m = (uint32_t)nearbyintf(scaled); /* FE_TONEAREST = ties to even */
    return (uint16_t)(sign | m);
  }
  const uint32_t e = (ax >> 23) - 127u + 15u;
  const uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may bump exponent */
  return (uint16_t)(sign | h);
}

static float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  float v;
  if (e == 0) {
    v = ldexpf((float)m, -24);
  } else if (e == 31) {
    v = m ? NAN : INFINITY;
  } else {
    v = ldexpf((float)(m | 0x400u), (int)e - 25);
  }
  uint32_t bits;
  memcpy(&bits, &v, 4);
  bits |= sign;
  memcpy(&v, &bits, 4);
  return v;
}

static uint16_t f32_to_bf16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u); /* quiet NaN */
  const uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return (uint16_t)(x >> 16);
}

static float bf16_bits_to_f32(uint16_t b) {
  const uint32_t x = (uint32_t)b << 16;
  float v;
  memcpy(&v, &x, 4);
  return v;
}

static float round_to(float x, int dtype) {
  return dtype == ORACLE_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x))
                              : f16_bits_to_f32(f32_to_f16_bits(x));
}

void oracle_round_f16(const float* in, float* out, uint16_t* bits, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const uint16_t h = f32_to_f16_bits(in[i]);
    if (bits) bits[i] = h;
    if (out) out[i] = f16_bits_to_f32(h);
  }
}

void oracle_round_bf16(const float* in, float* out, uint16_t* bits, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const uint16_t h = f32_to_bf16_bits(in[i]);
    if (bits) bits[i] = h;
    if (out) out[i] = bf16_bits_to_f32(h);
  }
}

/* ------------------------------------------------------------------------ */
/* exact fp64 oracle                                                        */
/* ------------------------------------------------------------------------ */

/* One query row i of head `bh`.  s_j = scale * q_i . k_j over visible keys. */
static void row_f64(const float* q, const float* k, const float* v, int N, int D, double scale,
                    int causal, int mutation, int i, double* s, double* o_row, double* lse) {
  const double sc = (mutation == ORACLE_MUT_NO_SCALE) ? 1.0 : scale;
  int jmax = N; /* keys [0, jmax) are visible */
  if (causal) jmax = (mutation == ORACLE_MUT_CAUSAL_DIAG) ? i : i + 1;
  double m = -INFINITY;
  for (int j = 0; j < jmax; ++j) {
    const float* qr = q + (int64_t)((mutation == ORACLE_MUT_TRANSPOSE_S) ? j : i) * D;
    const float* kr = k + (int64_t)((mutation == ORACLE_MUT_TRANSPOSE_S) ? i : j) * D;
    double acc = 0.0;
    for (int d = 0; d < D; ++d) acc = fma((double)qr[d], (double)kr[d], acc);
    s[j] = sc * acc;
    if (s[j] > m) m = s[j];
  }
  for (int d = 0; d < D; ++d) o_row[d] = 0.0;
  if (jmax == 0) { /* no visible key: O = 0, LSE = -inf */
    *lse = -INFINITY;
    return;
  }
  double l = 0.0;
  for (int j = 0; j < jmax; ++j) {
    const double p = exp(s[j] - m);
    l += p;
    const float* vr = v + (int64_t)j * D;
    for (int d = 0; d < D; ++d) o_row[d] = fma(p, (double)vr[d], o_row[d]);
  }
  if (mutation != ORACLE_MUT_NO_NORMALISE)
    for (int d = 0; d < D; ++d) o_row[d] /= l;
  *lse = (mutation == ORACLE_MUT_LSE_NO_MAX) ? log(l) : m + log(l);
}

int oracle_attn_rows_f64(const float* q, const float* k, const float* v, int B, int H, int N,
                         int D, double scale, int causal, int mutation, const int32_t* sel_bh,
                         const int32_t* sel_row, int64_t n_sel, double* o_sel, double* lse_sel) {
  if (B < 1 || H < 1 || N < 1 || D < 1) return -1;
  for (int64_t r = 0; r < n_sel; ++r)
    if (sel_bh[r] < 0 || sel_bh[r] >= B * H || sel_row[r] < 0 || sel_row[r] >= N) return -2;
  int err = 0;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)N);
    if (!s) {
#pragma omp atomic write
      err = -3;
    } else {
#pragma omp for schedule(dynamic, 4)
      for (int64_t r = 0; r < n_sel; ++r) {
        const int64_t off = (int64_t)sel_bh[r] * N * D;
        row_f64(q + off, k + off, v + off, N, D, scale, causal, mutation, sel_row[r], s,
                o_sel + r * D, lse_sel + r);
      }
      free(s);
    }
  }
  return err;
}

/* Rows [i0, i0 + nr) of one head at once (nr <= ORACLE_RB), mutation 0.
 * A single row's dot product is one dependent chain of D fused
 * multiply-adds, which leaves the FMA units mostly idle; a block of rows
 * against the same key gives ORACLE_RB independent chains.  Each row keeps
 * row_f64's arithmetic exactly (dot over d ascending, max, exp, l and O
 * summed over j ascending, all with explicit fma), so every output equals
 * row_f64's bit for bit (tests/test_oracle.py checks this).
 * Scratch: qt holds D x ORACLE_RB doubles, s ORACLE_RB x N. */
#define ORACLE_RB 16
static void rows_block_f64(const float* q, const float* k, const float* v, int N, int D,
                           double scale, int causal, int i0, int nr, double* qt, double* s,
                           double* o_rows, double* lse_rows) {
  for (int d = 0; d < D; ++d)
    for (int r = 0; r < ORACLE_RB; ++r)
      qt[d * ORACLE_RB + r] = r < nr ? (double)q[(int64_t)(i0 + r) * D + d] : 0.0;
  /* keys [0, jend) are visible to some row of the block */
  const int jend = causal ? (i0 + nr < N ? i0 + nr : N) : N;
  int j = 0;
  /* two keys x 16 rows: 8 independent 4-wide fma chains */
  for (; j + 1 < jend; j += 2) {
    const float* k0 = k + (int64_t)j * D;
    const float* k1 = k0 + D;
    __m256d a[2][4];
    for (int u = 0; u < 4; ++u) a[0][u] = a[1][u] = _mm256_setzero_pd();
    for (int d = 0; d < D; ++d) {
      const __m256d x0 = _mm256_set1_pd((double)k0[d]), x1 = _mm256_set1_pd((double)k1[d]);
      const double* qd = qt + d * ORACLE_RB;
      for (int u = 0; u < 4; ++u) {
        const __m256d qv = _mm256_loadu_pd(qd + 4 * u);
        a[0][u] = _mm256_fmadd_pd(qv, x0, a[0][u]);
        a[1][u] = _mm256_fmadd_pd(qv, x1, a[1][u]);
      }
    }
    double a0[ORACLE_RB], a1[ORACLE_RB];
    for (int u = 0; u < 4; ++u) {
      _mm256_storeu_pd(a0 + 4 * u, a[0][u]);
      _mm256_storeu_pd(a1 + 4 * u, a[1][u]);
    }
    for (int r = 0; r < ORACLE_RB; ++r) {
      s[(int64_t)r * N + j] = scale * a0[r];
      s[(int64_t)r * N + j + 1] = scale * a1[r];
    }
  }
  for (; j < jend; ++j) {
    const float* k0 = k + (int64_t)j * D;
    double a0[ORACLE_RB];
    for (int r = 0; r < ORACLE_RB; ++r) a0[r] = 0.0;
    for (int d = 0; d < D; ++d) {
      const double x0 = (double)k0[d];
      const double* qd = qt + d * ORACLE_RB;
      for (int r = 0; r < ORACLE_RB; ++r) a0[r] = fma(qd[r], x0, a0[r]);
    }
    for (int r = 0; r < ORACLE_RB; ++r) s[(int64_t)r * N + j] = scale * a0[r];
  }
  double l[ORACLE_RB];
  int jmax[ORACLE_RB];
  for (int r = 0; r < nr; ++r) {
    double* sr = s + (int64_t)r * N;
    jmax[r] = causal ? i0 + r + 1 : N;
    double m = -INFINITY;
    for (int jj = 0; jj < jmax[r]; ++jj)
      if (sr[jj] > m) m = sr[jj];
    double lr = 0.0;
    for (int jj = 0; jj < jmax[r]; ++jj) {
      sr[jj] = exp(sr[jj] - m); /* p_j, in place */
      lr += sr[jj];
    }
    l[r] = lr;
    lse_rows[r] = m + log(lr);
    for (int d = 0; d < D; ++d) o_rows[(int64_t)r * D + d] = 0.0;
  }
  for (int jj = 0; jj < jend; ++jj) {
    const float* vr = v + (int64_t)jj * D;
    for (int r = 0; r < nr; ++r) {
      if (jj >= jmax[r]) continue;
      const double p = s[(int64_t)r * N + jj];
      double* orow = o_rows + (int64_t)r * D;
      for (int d = 0; d < D; ++d) orow[d] = fma(p, (double)vr[d], orow[d]);
    }
  }
  for (int r = 0; r < nr; ++r)
    for (int d = 0; d < D; ++d) o_rows[(int64_t)r * D + d] /= l[r];
}

int oracle_attn_f64(const float* q, const float* k, const float* v, double* o, double* lse, int B,
                    int H, int N, int D, double scale, int causal, int mutation) {
  if (B < 1 || H < 1 || N < 1 || D < 1) return -1;
  int err = 0;
  if (mutation != ORACLE_MUT_NONE) {
    /* planted mistakes (small test shapes only): one row at a time */
#pragma omp parallel
    {
      double* s = (double*)malloc(sizeof(double) * (size_t)N);
      if (!s) {
#pragma omp atomic write
        err = -3;
      } else {
#pragma omp for schedule(dynamic, 4) collapse(2)
        for (int bh = 0; bh < B * H; ++bh)
          for (int i = 0; i < N; ++i) {
            const int64_t off = (int64_t)bh * N * D;
            row_f64(q + off, k + off, v + off, N, D, scale, causal, mutation, i, s,
                    o + off + (int64_t)i * D, lse + (int64_t)bh * N + i);
          }
        free(s);
      }
    }
    return err;
  }
  const int nblk = (N + ORACLE_RB - 1) / ORACLE_RB;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)N * ORACLE_RB);
    double* qt = (double*)malloc(sizeof(double) * (size_t)D * ORACLE_RB);
    if (!s || !qt) {
#pragma omp atomic write
      err = -3;
    } else {
      /* longest causal blocks (the last ones) first */
#pragma omp for schedule(dynamic, 1) collapse(2)
      for (int bi = 0; bi < nblk; ++bi)
        for (int bh = 0; bh < B * H; ++bh) {
          const int blk = nblk - 1 - bi;
          const int i0 = blk * ORACLE_RB;
          const int nr = N - i0 < ORACLE_RB ? N - i0 : ORACLE_RB;
          const int64_t off = (int64_t)bh * N * D;
          rows_block_f64(q + off, k + off, v + off, N, D, scale, causal, i0, nr, qt, s,
                         o + off + (int64_t)i0 * D, lse + (int64_t)bh * N + i0);
        }
    }
    free(s);
    free(qt);
  }
  return err;
}

/* ------------------------------------------------------------------------ */
/* the reference CPU path: fp32 online softmax with expf                    */
/* ------------------------------------------------------------------------ */

int oracle_ref_online_f32(const float* q, const float* k, const float* v, float* o, int B, int H,
                          int N, int D, float scale, int causal, int64_t row_begin,
                          int64_t row_end) {
  if (B < 1 || H < 1 || N < 1 || D < 1) return -1;
  const int64_t total = (int64_t)B * H * N;
  if (row_end > total) row_end = total;
  if (row_begin < 0) row_begin = 0;
  int err = 0;
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
    if (!acc) {
#pragma omp atomic write
      err = -3;
    } else {
#pragma omp for schedule(static)
      for (int64_t r = row_begin; r < row_end; ++r) {
        const int64_t bh = r / N;
        const int i = (int)(r - bh * N);
        const float* qb = q + bh * N * D;
        const float* kb = k + bh * N * D;
        const float* vb = v + bh * N * D;
        float m = -INFINITY, l = 0.0f;
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int j = 0; j < N; ++j) {
          float s = 0.0f;
          for (int d = 0; d < D; ++d) s += qb[(int64_t)i * D + d] * kb[(int64_t)j * D + d];
          s *= scale;
          if (causal && j > i) s = -INFINITY;
          const float m_new = fmaxf(m, s);
          if (m_new == -INFINITY) continue; /* nothing visible yet */
          const float alpha = expf(m - m_new);
          const float p = expf(s - m_new);
          for (int d = 0; d < D; ++d) acc[d] = acc[d] * alpha + p * vb[(int64_t)j * D + d];
          l = l * alpha + p;
          m = m_new;
        }
        const float inv_l = 1.0f / l;
        for (int d = 0; d < D; ++d) o[r * D + d] = acc[d] * inv_l;
      }
      free(acc);
    }
  }
  return err;
}

/* ------------------------------------------------------------------------ */
/* emulation of the reference kernel's numerics                             */
/* ------------------------------------------------------------------------ */

/* One query row i of head bh (q/k/v point at that head).  acc: D floats,
 * s: block_n floats of scratch. */
static void row_kernel_numerics(const float* qh, const float* kb, const float* vb, int N, int D,
                                float scale, int causal, int dtype, int block_n, int i,
                                float* acc, float* s, float* orow, float* lse) {
  const float c = scale * 1.4426950408889634f; /* config.cuh:84 */
  const float* qr = qh + (int64_t)i * D;
  float m = -INFINITY, l = 0.0f;
  for (int d = 0; d < D; ++d) acc[d] = 0.0f;
  for (int t0 = 0; t0 < N; t0 += block_n) {
    const int t1 = t0 + block_n < N ? t0 + block_n : N;
    if (causal && t0 > i) break; /* fully masked tile: skipped */
    float mt = m;
    for (int j = t0; j < t1; ++j) {
      float dot = 0.0f;
      for (int d = 0; d < D; ++d) dot = fmaf(qr[d], kb[(int64_t)j * D + d], dot);
      s[j - t0] = (causal && j > i) ? -INFINITY : dot;
      mt = fmaxf(mt, s[j - t0]);
    }
    const float m_use = mt == -INFINITY ? 0.0f : mt;
    const float alpha = exp2f((m - m_use) * c); /* online_softmax.cuh:17-19 */
    l *= alpha;
    for (int d = 0; d < D; ++d) acc[d] *= alpha;
    for (int j = t0; j < t1; ++j) {
      const float p = exp2f(fmaf(s[j - t0], c, -(m_use * c))); /* :13-15 */
      l += p;                                           /* unrounded p (:135-152) */
      const float pr = round_to(p, dtype);              /* P -> fp16/bf16 RNE */
      for (int d = 0; d < D; ++d) acc[d] = fmaf(pr, vb[(int64_t)j * D + d], acc[d]);
    }
    m = mt;
  }
  const float inv_l = 1.0f / l;
  for (int d = 0; d < D; ++d) orow[d] = round_to(acc[d] * inv_l, dtype);
  if (lse) *lse = (m == -INFINITY ? 0.0f : m) * scale + logf(l);
}

/* The emulation for rows [i0, i0 + nr) of one head at once (nr <=
 * ORACLE_RB), for the same reason as rows_block_f64: the rows' score dot
 * products against one key are independent chains.  Each row keeps
 * row_kernel_numerics' arithmetic exactly, so every output equals it bit for
 * bit.  Scratch: qt D x ORACLE_RB floats, s ORACLE_RB x block_n, acc
 * ORACLE_RB x D. */
static void rows_block_kernel_numerics(const float* qh, const float* kb, const float* vb, int N,
                                       int D, float scale, int causal, int dtype, int block_n,
                                       int i0, int nr, float* qt, float* s, float* acc,
                                       float* o_rows, float* lse_rows) {
  const float c = scale * 1.4426950408889634f; /* config.cuh:84 */
  for (int d = 0; d < D; ++d)
    for (int r = 0; r < ORACLE_RB; ++r)
      qt[d * ORACLE_RB + r] = r < nr ? qh[(int64_t)(i0 + r) * D + d] : 0.0f;
  float m[ORACLE_RB], l[ORACLE_RB];
  for (int r = 0; r < ORACLE_RB; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
  }
  for (int64_t x = 0; x < (int64_t)ORACLE_RB * D; ++x) acc[x] = 0.0f;
  for (int t0 = 0; t0 < N; t0 += block_n) {
    const int t1 = t0 + block_n < N ? t0 + block_n : N;
    if (causal && t0 > i0 + nr - 1) break; /* masked for every row of the block */
    int j = t0;
    /* four keys x 16 rows: 8 independent 8-wide fma chains */
    for (; j + 3 < t1; j += 4) {
      const float* kr = kb + (int64_t)j * D;
      __m256 a[4][2];
      for (int u = 0; u < 4; ++u) a[u][0] = a[u][1] = _mm256_setzero_ps();
      for (int d = 0; d < D; ++d) {
        const float* qd = qt + d * ORACLE_RB;
        const __m256 q0 = _mm256_loadu_ps(qd), q1 = _mm256_loadu_ps(qd + 8);
        for (int u = 0; u < 4; ++u) {
          const __m256 x = _mm256_set1_ps(kr[(int64_t)u * D + d]);
          a[u][0] = _mm256_fmadd_ps(q0, x, a[u][0]);
          a[u][1] = _mm256_fmadd_ps(q1, x, a[u][1]);
        }
      }
      for (int u = 0; u < 4; ++u) {
        float au[ORACLE_RB];
        _mm256_storeu_ps(au, a[u][0]);
        _mm256_storeu_ps(au + 8, a[u][1]);
        for (int r = 0; r < ORACLE_RB; ++r) s[(int64_t)r * block_n + (j + u - t0)] = au[r];
      }
    }
    for (; j < t1; ++j) {
      const float* kr = kb + (int64_t)j * D;
      float a[ORACLE_RB];
      for (int r = 0; r < ORACLE_RB; ++r) a[r] = 0.0f;
      for (int d = 0; d < D; ++d) {
        const float x = kr[d];
        const float* qd = qt + d * ORACLE_RB;
        for (int r = 0; r < ORACLE_RB; ++r) a[r] = fmaf(qd[r], x, a[r]);
      }
      for (int r = 0; r < ORACLE_RB; ++r) s[(int64_t)r * block_n + (j - t0)] = a[r];
    }
    for (int r = 0; r < nr; ++r) {
      const int i = i0 + r;
      if (causal && t0 > i) continue; /* fully masked tile for this row: skipped */
      float* sr = s + (int64_t)r * block_n;
      float mt = m[r];
      for (int j = t0; j < t1; ++j) {
        if (causal && j > i) sr[j - t0] = -INFINITY;
        mt = fmaxf(mt, sr[j - t0]);
      }
      const float m_use = mt == -INFINITY ? 0.0f : mt;
      const float alpha = exp2f((m[r] - m_use) * c); /* online_softmax.cuh:17-19 */
      l[r] *= alpha;
      float* ar = acc + (int64_t)r * D;
      for (int d = 0; d < D; ++d) ar[d] *= alpha;
      for (int j = t0; j < t1; ++j) {
        const float p = exp2f(fmaf(sr[j - t0], c, -(m_use * c))); /* :13-15 */
        l[r] += p;                                               /* unrounded p (:135-152) */
        sr[j - t0] = round_to(p, dtype); /* P -> fp16/bf16 RNE, in place */
      }
      m[r] = mt;
    }
    for (int j = t0; j < t1; ++j) {
      const float* vr = vb + (int64_t)j * D;
      for (int r = 0; r < nr; ++r) {
        if (causal && t0 > i0 + r) continue;
        const float pr = s[(int64_t)r * block_n + (j - t0)];
        float* ar = acc + (int64_t)r * D;
        for (int d = 0; d < D; ++d) ar[d] = fmaf(pr, vr[d], ar[d]);
      }
    }
  }
  for (int r = 0; r < nr; ++r) {
    const float inv_l = 1.0f / l[r];
    for (int d = 0; d < D; ++d)
      o_rows[(int64_t)r * D + d] = round_to(acc[(int64_t)r * D + d] * inv_l, dtype);
    if (lse_rows) lse_rows[r] = (m[r] == -INFINITY ? 0.0f : m[r]) * scale + logf(l[r]);
  }
}

int oracle_kernel_numerics(const float* q, const float* k, const float* v, float* o, float* lse,
                           int B, int H, int N, int D, float scale, int causal, int dtype,
                           int block_n) {
  if (B < 1 || H < 1 || N < 1 || D < 1 || block_n < 1) return -1;
  int err = 0;
  const int nblk = (N + ORACLE_RB - 1) / ORACLE_RB;
#pragma omp parallel
  {
    float* qt = (float*)malloc(sizeof(float) * (size_t)D * ORACLE_RB);
    float* s = (float*)malloc(sizeof(float) * (size_t)block_n * ORACLE_RB);
    float* acc = (float*)malloc(sizeof(float) * (size_t)D * ORACLE_RB);
    if (!qt || !s || !acc) {
#pragma omp atomic write
      err = -3;
    } else {
#pragma omp for schedule(dynamic, 1) collapse(2)
      for (int bi = 0; bi < nblk; ++bi)
        for (int bh = 0; bh < B * H; ++bh) {
          const int blk = nblk - 1 - bi; /* longest causal blocks first */
          const int i0 = blk * ORACLE_RB;
          const int nr = N - i0 < ORACLE_RB ? N - i0 : ORACLE_RB;
          const int64_t off = (int64_t)bh * N * D;
          rows_block_kernel_numerics(q + off, k + off, v + off, N, D, scale, causal, dtype,
                                     block_n, i0, nr, qt, s, acc, o + off + (int64_t)i0 * D,
                                     lse ? lse + (int64_t)bh * N + i0 : NULL);
        }
    }
    free(qt);
    free(s);
    free(acc);
  }
  return err;
}

int oracle_kernel_numerics_rows(const float* q, const float* k, const float* v, int B, int H,
                                int N, int D, float scale, int causal, int dtype, int block_n,
                                const int32_t* sel_bh, const int32_t* sel_row, int64_t n_sel,
                                float* o_sel, float* lse_sel) {
  if (B < 1 || H < 1 || N < 1 || D < 1 || block_n < 1) return -1;
  for (int64_t r = 0; r < n_sel; ++r)
    if (sel_bh[r] < 0 || sel_bh[r] >= B * H || sel_row[r] < 0 || sel_row[r] >= N) return -2;
  int err = 0;
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
    float* s = (float*)malloc(sizeof(float) * (size_t)block_n);
    if (!acc || !s) {
#pragma omp atomic write
      err = -3;
    } else {
#pragma omp for schedule(dynamic, 4)
      for (int64_t r = 0; r < n_sel; ++r) {
        const int64_t off = (int64_t)sel_bh[r] * N * D;
        row_kernel_numerics(q + off, k + off, v + off, N, D, scale, causal, dtype, block_n,
                            sel_row[r], acc, s, o_sel + r * D, lse_sel + r);
      }
    }
    free(acc);
    free(s);
  }
  return err;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
