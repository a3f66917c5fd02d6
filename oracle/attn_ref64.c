/*
 * Float64 brute-force attention: TEST INFRASTRUCTURE ONLY (never linked into the product).
 *
 * Restates the reference's double-precision CPU check, /root/reference/sim/harness.cu:40-64:
 * for every (bh, query row i) compute s_j = (q_i . k_j) / sqrt(d) in double (keys j > i
 * masked when causal), subtract the row max, exponentiate, and form sum_j p_j v_j / sum_j p_j.
 * Inputs are float32 arrays laid out [BH][N][d] (fp16/bf16 inputs are widened by the caller);
 * the output is float64 [BH][N][d]. Rows are independent, so they are split across OpenMP
 * threads. Used by tests to pin oracle/online_softmax.py:attention_naive with a second,
 * independently written implementation.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

int attn_ref64(const float* q, const float* k, const float* v, double* o,
               int64_t BH, int64_t N, int64_t d, int causal) {
  if (BH < 0 || N < 0 || d <= 0) return 1;
  const double scale = 1.0 / sqrt((double)d);
  int fail = 0;
#pragma omp parallel
  {
    double* s = (double*)malloc((size_t)(N > 0 ? N : 1) * sizeof(double));
    double* acc = (double*)malloc((size_t)d * sizeof(double));
    if (!s || !acc) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t row = 0; row < BH * N; ++row) {
        const int64_t bh = row / N, i = row % N;
        const float* qi = q + row * d;
        const int64_t jend = causal ? i + 1 : N;
        double m = -INFINITY;
        for (int64_t j = 0; j < jend; ++j) {
          const float* kj = k + (bh * N + j) * d;
          double dot = 0.0;
          for (int64_t c = 0; c < d; ++c) dot += (double)qi[c] * (double)kj[c];
          s[j] = dot * scale;
          if (s[j] > m) m = s[j];
        }
        double l = 0.0;
        for (int64_t c = 0; c < d; ++c) acc[c] = 0.0;
        for (int64_t j = 0; j < jend; ++j) {
          const double p = exp(s[j] - m);
          l += p;
          const float* vj = v + (bh * N + j) * d;
          for (int64_t c = 0; c < d; ++c) acc[c] += p * (double)vj[c];
        }
        double* oi = o + row * d;
        for (int64_t c = 0; c < d; ++c) oi[c] = acc[c] / l;
      }
    }
    free(s);
    free(acc);
  }
  return fail;
}
