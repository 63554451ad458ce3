/*
 * fp64 loop restatement of the dense hot path.  TEST INFRASTRUCTURE ONLY:
 * loaded by tests/ (through oracle/native.py) as an independent second oracle
 * next to the numpy restatement in reference.py; never linked into the product.
 *
 * oracle_gemm       C = A @ B with arbitrary strides (DotTests.swift:16-30)
 * oracle_attention  O, log2-LSE, Delta, dQ, dK, dV and the cancellation
 *                   amplification, from the definitions
 *                   (AttentionBackwardTests.swift:46-160), plus a causal mask
 *                   (key > query excluded) that the reference does not have.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

void oracle_gemm(const float *a, const float *b, double *c, int m, int n, int k, int sam,
                 int sak, int sbk, int sbn) {
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int t = 0; t < k; ++t)
        acc += (double)a[(long)i * sam + (long)t * sak] * (double)b[(long)t * sbk + (long)j * sbn];
      c[(long)i * n + j] = acc;
    }
}

static double fmax_d(double a, double b) { return a > b ? a : b; }

int oracle_attention(const float *q, const float *k, const float *v, const float *dout,
                     int heads, int seq, int dim, double scale, int causal, double *o,
                     double *lse2, double *delta, double *dq, double *dk, double *dv,
                     double *amplification) {
  const double log2e = 1.4426950408889634;
  double *prob = (double *)malloc(sizeof(double) * (size_t)seq * seq);
  double *ds = (double *)malloc(sizeof(double) * (size_t)seq * seq);
  if (!prob || !ds) {
    free(prob);
    free(ds);
    return -1;
  }
  double dq_terms = 0, dk_terms = 0, dv_terms = 0;
  double dq_peak = 0, dk_peak = 0, dv_peak = 0;
  for (int h = 0; h < heads; ++h) {
    const long base = (long)h * seq * dim;
    for (int i = 0; i < seq; ++i) {
      const int last = causal ? i : seq - 1;
      double peak = -INFINITY;
      for (int j = 0; j <= last; ++j) {
        double s = 0;
        for (int d = 0; d < dim; ++d)
          s += (double)q[base + (long)i * dim + d] * (double)k[base + (long)j * dim + d];
        s *= scale;
        prob[(long)i * seq + j] = s;
        peak = fmax_d(peak, s);
      }
      double sum = 0;
      for (int j = 0; j < seq; ++j) {
        if (j <= last) {
          prob[(long)i * seq + j] = exp(prob[(long)i * seq + j] - peak);
          sum += prob[(long)i * seq + j];
        } else {
          prob[(long)i * seq + j] = 0;
        }
      }
      for (int j = 0; j <= last; ++j) prob[(long)i * seq + j] /= sum;
      lse2[(long)h * seq + i] = peak * log2e + log2(sum);
      for (int d = 0; d < dim; ++d) {
        double acc = 0;
        for (int j = 0; j <= last; ++j)
          acc += prob[(long)i * seq + j] * (double)v[base + (long)j * dim + d];
        o[base + (long)i * dim + d] = acc;
      }
      double dd = 0;
      for (int d = 0; d < dim; ++d)
        dd += (double)dout[base + (long)i * dim + d] * o[base + (long)i * dim + d];
      delta[(long)h * seq + i] = dd;
    }
    for (int i = 0; i < seq; ++i)
      for (int j = 0; j < seq; ++j) {
        double dp = 0;
        for (int d = 0; d < dim; ++d)
          dp += (double)dout[base + (long)i * dim + d] * (double)v[base + (long)j * dim + d];
        ds[(long)i * seq + j] = prob[(long)i * seq + j] * (dp - delta[(long)h * seq + i]);
      }
    for (int i = 0; i < seq; ++i)
      for (int d = 0; d < dim; ++d) {
        double total = 0, absolute = 0;
        for (int j = 0; j < seq; ++j) {
          const double term = ds[(long)i * seq + j] * (double)k[base + (long)j * dim + d] * scale;
          total += term;
          absolute += fabs(term);
        }
        dq[base + (long)i * dim + d] = total;
        dq_terms = fmax_d(dq_terms, absolute);
        dq_peak = fmax_d(dq_peak, fabs(total));
      }
    for (int j = 0; j < seq; ++j)
      for (int d = 0; d < dim; ++d) {
        double tk = 0, ak = 0, tv = 0, av = 0;
        for (int i = 0; i < seq; ++i) {
          const double term_k = ds[(long)i * seq + j] * (double)q[base + (long)i * dim + d] * scale;
          const double term_v = prob[(long)i * seq + j] * (double)dout[base + (long)i * dim + d];
          tk += term_k;
          ak += fabs(term_k);
          tv += term_v;
          av += fabs(term_v);
        }
        dk[base + (long)j * dim + d] = tk;
        dv[base + (long)j * dim + d] = tv;
        dk_terms = fmax_d(dk_terms, ak);
        dv_terms = fmax_d(dv_terms, av);
        dk_peak = fmax_d(dk_peak, fabs(tk));
        dv_peak = fmax_d(dv_peak, fabs(tv));
      }
  }
  amplification[0] = dq_terms / fmax_d(dq_peak, 1e-30);
  amplification[1] = dk_terms / fmax_d(dk_peak, 1e-30);
  amplification[2] = dv_terms / fmax_d(dv_peak, 1e-30);
  free(prob);
  free(ds);
  return 0;
}
