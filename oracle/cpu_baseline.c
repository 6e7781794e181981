/* cpu_baseline.c -- OpenMP fp32 CPU path of the five hot-path operators.
 *
 * TEST INFRASTRUCTURE ONLY: this is the timed CPU baseline that bench.py
 * reports next to the GPU numbers (and a second, independent CPU restatement
 * for the tests).  The product never links or calls it.
 *
 * It restates the reference's own CPU execution model, a100c's worker pool:
 * program instances (rows, or output tiles) are dealt to W workers in the
 * strided order of a100c/plan/partition.py:26-35 (worker w runs programs
 * w, w+W, ...) -- OpenMP schedule(static, 1) -- with fp32 accumulation as the
 * reference lowering uses for 16-bit inputs (a100c/lower/vectorize.py:9578-9592).
 * Operator formulas: softmax ops/suite/perf/softmax.py:21-32; RMSNorm
 * ops/suite/perf/fast_rms_layernorm.py:20-42; LayerNorm
 * ops/suite/dev/fused_layernorm_triton.py:27-42; GEMM ops/suite/perf/matmul.py:21-37;
 * attention ops/suite/perf/attn_fwd_causal.py:20-55 with GQA (ops/suite/dev/gqa.py:29)
 * and LSE (ops/suite/dev/flash_varlen_fwd_kernel.py:309).
 * bf16 is carried as uint16 bits; narrowing is round-to-nearest-even with
 * NaN quieting (ops/harness/opslib/case.py:214-220).
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t tobf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) r = u | 0x00400000u;
  return (uint16_t)(r >> 16);
}

int g950o_threads(void) {
  int n = 1;
#pragma omp parallel
  {
#pragma omp single
    n = omp_get_num_threads();
  }
  return n;
}

void g950o_softmax_f32(const float *x, float *y, long rows, long cols) {
#pragma omp parallel for schedule(static, 1)
  for (long r = 0; r < rows; ++r) {
    const float *xr = x + r * cols;
    float *yr = y + r * cols;
    float m = -INFINITY;
    for (long j = 0; j < cols; ++j) m = xr[j] > m ? xr[j] : m;
    float s = 0.0f;
    for (long j = 0; j < cols; ++j) {
      yr[j] = expf(xr[j] - m);
      s += yr[j];
    }
    const float inv = 1.0f / s;
    for (long j = 0; j < cols; ++j) yr[j] *= inv;
  }
}

void g950o_rmsnorm_f32(const float *x, const float *w, float *y, float *rr, long rows, long cols,
                       float eps) {
#pragma omp parallel for schedule(static, 1)
  for (long r = 0; r < rows; ++r) {
    const float *xr = x + r * cols;
    float ss = 0.0f;
#pragma omp simd reduction(+ : ss)
    for (long j = 0; j < cols; ++j) ss += xr[j] * xr[j];
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    rr[r] = inv;
    for (long j = 0; j < cols; ++j) y[r * cols + j] = (xr[j] * inv) * w[j];
  }
}

void g950o_softmax_bf16(const uint16_t *x, uint16_t *y, long rows, long cols) {
#pragma omp parallel
  {
    float *buf = (float *)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static, 1)
    for (long r = 0; r < rows; ++r) {
      const uint16_t *xr = x + r * cols;
      float m = -INFINITY;
      for (long j = 0; j < cols; ++j) {
        buf[j] = bf(xr[j]);
        m = buf[j] > m ? buf[j] : m;
      }
      float s = 0.0f;
      for (long j = 0; j < cols; ++j) {
        buf[j] = expf(buf[j] - m);
        s += buf[j];
      }
      const float inv = 1.0f / s;
      for (long j = 0; j < cols; ++j) y[r * cols + j] = tobf(buf[j] * inv);
    }
    free(buf);
  }
}

void g950o_layernorm_bf16(const uint16_t *x, const uint16_t *w, const uint16_t *b, uint16_t *y,
                          float *mean_out, float *rstd_out, long rows, long cols, float eps) {
#pragma omp parallel
  {
    float *buf = (float *)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static, 1)
    for (long r = 0; r < rows; ++r) {
      const uint16_t *xr = x + r * cols;
      float s = 0.0f;
      for (long j = 0; j < cols; ++j) {
        buf[j] = bf(xr[j]);
        s += buf[j];
      }
      const float mean = s / (float)cols;
      float q = 0.0f;
      for (long j = 0; j < cols; ++j) {
        buf[j] -= mean;
        q += buf[j] * buf[j];
      }
      const float rstd = 1.0f / sqrtf(q / (float)cols + eps);
      mean_out[r] = mean;
      rstd_out[r] = rstd;
      for (long j = 0; j < cols; ++j) y[r * cols + j] = tobf(buf[j] * rstd * bf(w[j]) + bf(b[j]));
    }
    free(buf);
  }
}

/* bf16 bits -> fp32 values (exact widening), n elements. */
void g950o_widen_bf16(const uint16_t *src, float *dst, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) dst[i] = bf(src[i]);
}

/* C[m, n] = sum_k A[m, k] * Bt[n, k] for rows [m0, m1) of bf16 A, with Bt
 * already widened to fp32; fp32 accumulate, bf16 output.  Tiles of 4 output
 * rows x 4 output columns are the programs. */
void g950o_gemm_bf16_wide(const uint16_t *a, const float *bf32, uint16_t *c, long m0, long m1, long N,
                          long K) {
  const long mt = (m1 - m0 + 3) / 4, nt = (N + 3) / 4;
#pragma omp parallel
  {
    float *arow = (float *)malloc(sizeof(float) * 4 * (size_t)K);
#pragma omp for schedule(static, 1)
    for (long t = 0; t < mt * nt; ++t) {
      const long ti = t / nt, tj = t % nt;
      const long mb = m0 + ti * 4, nb = tj * 4;
      for (int i = 0; i < 4; ++i)
        for (long k = 0; k < K; ++k) arow[i * K + k] = (mb + i < m1) ? bf(a[(mb + i) * K + k]) : 0.0f;
      for (int i = 0; i < 4 && mb + i < m1; ++i)
        for (int j = 0; j < 4 && nb + j < N; ++j) {
          const float *ar = arow + i * K, *br = bf32 + (nb + j) * K;
          float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
          for (long k = 0; k < K; ++k) acc += ar[k] * br[k];
          c[(mb + i - m0) * N + nb + j] = tobf(acc);
        }
    }
    free(arow);
  }
}

/* The same with Bt in bf16 (widened here first). */
void g950o_gemm_bf16(const uint16_t *a, const uint16_t *bt, uint16_t *c, long m0, long m1, long N,
                     long K) {
  float *bf32 = (float *)malloc(sizeof(float) * (size_t)N * (size_t)K);
  g950o_widen_bf16(bt, bf32, N * K);
  g950o_gemm_bf16_wide(a, bf32, c, m0, m1, N, K);
  free(bf32);
}

/* int8 GEMM rows [m0, m1): exact int32 accumulate, dequant epilogue. */
void g950o_gemm_i8(const int8_t *a, const int8_t *bt, const float *sa, const float *sb, int32_t *acc_out,
                   uint16_t *y, long m0, long m1, long N, long K) {
#pragma omp parallel for schedule(static, 1)
  for (long m = m0; m < m1; ++m) {
    const int8_t *ar = a + m * K;
    for (long n = 0; n < N; ++n) {
      const int8_t *br = bt + n * K;
      int32_t acc = 0;
#pragma omp simd reduction(+ : acc)
      for (long k = 0; k < K; ++k) acc += (int32_t)ar[k] * (int32_t)br[k];
      if (acc_out) acc_out[(m - m0) * N + n] = acc;
      y[(m - m0) * N + n] = tobf(((float)acc * sa[m]) * sb[n]);
    }
  }
}

/* Causal (or full) GQA attention for heads [h0, h1) of batch z and query rows
 * [q0, q1); q [Hq, S, D], k/v [Hkv, S, D] of that batch, contiguous bf16.
 * o [h1-h0, q1-q0, D] bf16, lse [h1-h0, q1-q0] fp32. */
void g950o_attention_bf16(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *o,
                          float *lse, long Hq, long Hkv, long S, long D, long h0, long h1, long q0,
                          long q1, float scale, int causal) {
  const long G = Hq / Hkv;
  const long nq = q1 - q0;
#pragma omp parallel
  {
    float *s = (float *)malloc(sizeof(float) * (size_t)S);
    float *acc = (float *)malloc(sizeof(float) * (size_t)D);
    float *qv = (float *)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(static, 1)
    for (long t = 0; t < (h1 - h0) * nq; ++t) {
      const long h = h0 + t / nq, i = q0 + t % nq;
      const uint16_t *qr = q + (h * S + i) * D;
      const uint16_t *kh = k + (h / G) * S * D, *vh = v + (h / G) * S * D;
      const long kend = causal ? i + 1 : S;
      for (long d = 0; d < D; ++d) qv[d] = bf(qr[d]);
      float m = -INFINITY;
      for (long j = 0; j < kend; ++j) {
        float dot = 0.0f;
        for (long d = 0; d < D; ++d) dot += qv[d] * bf(kh[j * D + d]);
        s[j] = dot * scale;
        m = s[j] > m ? s[j] : m;
      }
      float l = 0.0f;
      for (long d = 0; d < D; ++d) acc[d] = 0.0f;
      for (long j = 0; j < kend; ++j) {
        const float p = expf(s[j] - m);
        l += p;
        for (long d = 0; d < D; ++d) acc[d] += p * bf(vh[j * D + d]);
      }
      uint16_t *orow = o + ((h - h0) * nq + (i - q0)) * D;
      for (long d = 0; d < D; ++d) orow[d] = tobf(acc[d] / l);
      lse[(h - h0) * nq + (i - q0)] = m + logf(l);
    }
    free(s);
    free(acc);
    free(qv);
  }
}
