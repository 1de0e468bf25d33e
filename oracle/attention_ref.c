/*
 * attention_ref.c -- plain-C float64 brute-force attention, forward and
 * backward.  TEST INFRASTRUCTURE ONLY: loaded by tests/ as an independent
 * check of oracle/attention.py (explicit loops and a two-pass softmax here,
 * matrix products there), never by the product path.
 *
 * Semantics restated from the reference:
 *   forward  : flash_attn_volta/ref.py:9-36 (scores * sm_scale, causal strict
 *              upper triangle = -inf, softmax, P V) with the kernel's LSE
 *              contract triton_fa.py:152-159 (LSE = m + ln l, +inf if a row
 *              sees no key);
 *   backward : triton_fa_bwd.py:165-178 (P = exp(S - LSE), dP = dO V^T,
 *              dS = P (dP - delta), dQ = sm_scale dS K) and :415-429
 *              (dV = P^T dO, dK = sm_scale dS^T Q); delta = rowsum(O dO)
 *              over the O the caller passes (:649-650).
 * Layout: (B, S, H, D) contiguous float64; lse / delta (B, H, S).
 */
#include <math.h>
#include <stdlib.h>

static size_t idx(int b, int s, int h, int d, int S, int H, int D) {
  return (((size_t)b * S + s) * H + h) * D + d;
}

/* score of query i against key j, or -inf when masked */
static double score(const double *q, const double *k, int b, int h, int i, int j,
                    int S, int H, int D, double scale, int causal) {
  if (causal && j > i) return -INFINITY;
  double acc = 0.0;
  for (int d = 0; d < D; ++d) acc += q[idx(b, i, h, d, S, H, D)] * k[idx(b, j, h, d, S, H, D)];
  return acc * scale;
}

/* row i probabilities into p[0..S), returns the natural-log LSE */
static double row_probs(const double *q, const double *k, int b, int h, int i, int S, int H,
                        int D, double scale, int causal, double *p) {
  double m = -INFINITY;
  for (int j = 0; j < S; ++j) {
    p[j] = score(q, k, b, h, i, j, S, H, D, scale, causal);
    if (p[j] > m) m = p[j];
  }
  if (!isfinite(m)) {
    for (int j = 0; j < S; ++j) p[j] = 0.0;
    return INFINITY;
  }
  double l = 0.0;
  for (int j = 0; j < S; ++j) {
    p[j] = exp(p[j] - m);
    l += p[j];
  }
  for (int j = 0; j < S; ++j) p[j] /= l;
  return m + log(l);
}

int oracle_fwd(const double *q, const double *k, const double *v, int B, int S, int H, int D,
               double scale, int causal, double *o, double *lse) {
  double *p = (double *)malloc(sizeof(double) * (size_t)S);
  if (!p) return -1;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h)
      for (int i = 0; i < S; ++i) {
        lse[((size_t)b * H + h) * S + i] = row_probs(q, k, b, h, i, S, H, D, scale, causal, p);
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int j = 0; j < S; ++j) acc += p[j] * v[idx(b, j, h, d, S, H, D)];
          o[idx(b, i, h, d, S, H, D)] = acc;
        }
      }
  free(p);
  return 0;
}

/* o_given may be NULL: then the exact float64 forward output is used. */
int oracle_bwd(const double *dout, const double *q, const double *k, const double *v,
               const double *o_given, int B, int S, int H, int D, double scale, int causal,
               double *dq, double *dk, double *dv, double *delta) {
  const size_t n = (size_t)B * S * H * D;
  double *p = (double *)malloc(sizeof(double) * (size_t)S);
  double *o = (double *)malloc(sizeof(double) * n);
  double *lse = (double *)malloc(sizeof(double) * (size_t)B * H * S);
  if (!p || !o || !lse) {
    free(p); free(o); free(lse);
    return -1;
  }
  if (o_given) {
    for (size_t x = 0; x < n; ++x) o[x] = o_given[x];
  } else {
    oracle_fwd(q, k, v, B, S, H, D, scale, causal, o, lse);
  }
  for (size_t x = 0; x < n; ++x) dq[x] = dk[x] = dv[x] = 0.0;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h)
      for (int i = 0; i < S; ++i) {
        double dl = 0.0;
        for (int d = 0; d < D; ++d) dl += o[idx(b, i, h, d, S, H, D)] * dout[idx(b, i, h, d, S, H, D)];
        delta[((size_t)b * H + h) * S + i] = dl;
        row_probs(q, k, b, h, i, S, H, D, scale, causal, p);
        for (int j = 0; j < S; ++j) {
          if (p[j] == 0.0) continue;
          double dp = 0.0;
          for (int d = 0; d < D; ++d) dp += dout[idx(b, i, h, d, S, H, D)] * v[idx(b, j, h, d, S, H, D)];
          const double ds = p[j] * (dp - dl);
          for (int d = 0; d < D; ++d) {
            dq[idx(b, i, h, d, S, H, D)] += scale * ds * k[idx(b, j, h, d, S, H, D)];
            dk[idx(b, j, h, d, S, H, D)] += scale * ds * q[idx(b, i, h, d, S, H, D)];
            dv[idx(b, j, h, d, S, H, D)] += p[j] * dout[idx(b, i, h, d, S, H, D)];
          }
        }
      }
  free(p); free(o); free(lse);
  return 0;
}
