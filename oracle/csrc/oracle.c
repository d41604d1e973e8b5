/*
 * Scalar C restatement of the reference math, in double precision loops:
 * TEST INFRASTRUCTURE ONLY (the oracle's second, independent statement; the
 * tests check the torch oracle against it on small inputs).
 *
 * Each function cites the reference file:line it restates.
 */
#include <math.h>
#include <stdint.h>

/* kernels/cumsum/refs.py:20-22 (torch.cumsum: double accumulation, one
 * rounding per prefix). */
void oracle_cumsum_rows(const float* x, float* y, int64_t m, int64_t n) {
  for (int64_t i = 0; i < m; ++i) {
    double acc = 0.0;
    for (int64_t j = 0; j < n; ++j) {
      acc += (double)x[i * n + j];
      y[i * n + j] = (float)acc;
    }
  }
}

/* kernels/rmsnorm/refs.py:21-30: x / sqrt(sum x^2) (mode 0), and the
 * mean/eps/weight form x * rsqrt(mean x^2 + eps) * w (mode 1). */
void oracle_rmsnorm_rows(const float* x, const float* w, float* y, int64_t m, int64_t n,
                         int mode, double eps) {
  for (int64_t i = 0; i < m; ++i) {
    double s = 0.0;
    for (int64_t j = 0; j < n; ++j) s += (double)x[i * n + j] * (double)x[i * n + j];
    const double scale = mode == 0 ? 1.0 / sqrt(s) : 1.0 / sqrt(s / (double)n + eps);
    for (int64_t j = 0; j < n; ++j)
      y[i * n + j] = (float)((double)x[i * n + j] * scale * (mode == 0 ? 1.0 : (double)w[j]));
  }
}

/* kernels/layernorm/refs.py:16-37. */
void oracle_layernorm_rows(const float* x, float* y, int64_t m, int64_t n, double eps) {
  for (int64_t i = 0; i < m; ++i) {
    double s = 0.0;
    for (int64_t j = 0; j < n; ++j) s += x[i * n + j];
    const double mean = s / (double)n;
    double q = 0.0;
    for (int64_t j = 0; j < n; ++j) q += ((double)x[i * n + j] - mean) * ((double)x[i * n + j] - mean);
    const double inv = 1.0 / sqrt(q / (double)n + eps);
    for (int64_t j = 0; j < n; ++j) y[i * n + j] = (float)(((double)x[i * n + j] - mean) * inv);
  }
}

/* kernels/softmax/kernel.py:13-16 (no max shift). */
void oracle_softmax_rows(const float* x, float* y, int64_t m, int64_t n) {
  for (int64_t i = 0; i < m; ++i) {
    double s = 0.0;
    for (int64_t j = 0; j < n; ++j) s += exp((double)x[i * n + j]);
    for (int64_t j = 0; j < n; ++j) y[i * n + j] = (float)(exp((double)x[i * n + j]) / s);
  }
}

/* Rotate-half RoPE on token-major x[t][h][d] with cos/sin[t % s][d]
 * (kernels/rope/kernel.py:33-36 with x_even = x[:d/2], x_odd = x[d/2:]). */
void oracle_rope_rotate_half(const float* x, const float* c, const float* sn, float* y,
                             int64_t tokens, int64_t s, int64_t heads, int64_t d) {
  const int64_t half = d / 2;
  for (int64_t t = 0; t < tokens; ++t)
    for (int64_t hh = 0; hh < heads; ++hh) {
      const float* xr = x + (t * heads + hh) * d;
      float* yr = y + (t * heads + hh) * d;
      const float* cr = c + (t % s) * d;
      const float* sr = sn + (t % s) * d;
      for (int64_t i = 0; i < half; ++i) {
        const double a = xr[i], b = xr[i + half];
        yr[i] = (float)(a * cr[i] - b * sr[i]);
        yr[i + half] = (float)(b * cr[i + half] + a * sr[i + half]);
      }
    }
}

/* kernels/fused_adam/refs.py:38-46, each operation rounded to fp32 in the
 * reference's order (this file is built with -ffp-contract=off). */
void oracle_fused_adam(const float* p, const float* g, const float* m, const float* v,
                       const float* step, const float* ibc, const float* wd, float* po, float* mo,
                       float* vo, int64_t rows, int64_t f) {
  const float b1 = (float)0.9, omb1 = (float)(1.0 - 0.9);
  const float b2 = (float)0.999, omb2 = (float)(1.0 - 0.999);
  const float eps = (float)1e-8;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < f; ++j) {
      const int64_t i = r * f + j;
      const float gp = g[i] + wd[r] * p[i];
      const float mn = b1 * m[i] + omb1 * gp;
      const float vn = b2 * v[i] + omb2 * (gp * gp);
      const float den = sqrtf(vn) * ibc[r] + eps;
      po[i] = p[i] - mn / den * step[r];
      mo[i] = mn;
      vo[i] = vn;
    }
}

/* x[m,k] @ w[k,n] in double (kernels/matmul/refs.py:20-25). */
void oracle_matmul_f64(const float* x, const float* w, double* y, int64_t m, int64_t n, int64_t k) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double s = 0.0;
      for (int64_t q = 0; q < k; ++q) s += (double)x[i * k + q] * (double)w[q * n + j];
      y[i * n + j] = s;
    }
}

/* Causal softmax(q k^T * scale) v for one head, in double
 * (kernels/attention_nkilib/kernel.py:14-21 with scale and mask). */
void oracle_attention_head_f64(const float* q, const float* k, const float* v, double* o,
                               int64_t s, int64_t d, double scale, int causal) {
  for (int64_t i = 0; i < s; ++i) {
    double mx = -INFINITY;
    const int64_t last = causal ? i : s - 1;
    for (int64_t j = 0; j <= last; ++j) {
      double dot = 0.0;
      for (int64_t t = 0; t < d; ++t) dot += (double)q[i * d + t] * (double)k[j * d + t];
      dot *= scale;
      if (dot > mx) mx = dot;
    }
    double den = 0.0;
    for (int64_t t = 0; t < d; ++t) o[i * d + t] = 0.0;
    for (int64_t j = 0; j <= last; ++j) {
      double dot = 0.0;
      for (int64_t t = 0; t < d; ++t) dot += (double)q[i * d + t] * (double)k[j * d + t];
      const double p = exp(dot * scale - mx);
      den += p;
      for (int64_t t = 0; t < d; ++t) o[i * d + t] += p * (double)v[j * d + t];
    }
    for (int64_t t = 0; t < d; ++t) o[i * d + t] /= den;
  }
}
