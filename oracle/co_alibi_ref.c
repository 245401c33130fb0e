/*
 * Plain-C restatement of Co-ALiBi attention -- TEST INFRASTRUCTURE ONLY (see co_alibi_ref.h).
 *
 * Follows the reference's PyTorch algorithm, model.py:13-76, with the per-head slope its
 * kernels and validation scripts apply (co_alibi_attn/co_alibi_attn.py:147,
 * benchmark_bwd_pass.py:89-91), the non-causal mode of co_alibi_fwd_kernel.py:80-90 and the
 * grouped-query head mapping of co_alibi_attn.py:143-146.  Per query row i of head h:
 *   p_j   = scale * q_i . k_j                                        model.py:15
 *   s_j   = sigmoid(p_j) on visible keys, else 0                     model.py:23
 *   z_j   = sum over keys k >= j of s_k                              model.py:24
 *   a_j   = p_j - slope_h * z_j                                      model.py:26-27
 *   w_j   = exp(a_j - max a) on visible keys, l = sum w + 1e-9       model.py:29-36
 *   O     = sum_j (w_j / l) v_j,   LSE = max a + log l               model.py:38-40, fwd:120
 * and the backward (model.py:57-76): with P_j = w_j / l,
 *   dv_j += P_j dO,   dS_j = dO . v_j,   dsum = sum_j dS_j P_j,   dA_j = P_j (dS_j - dsum),
 *   C_j = sum over keys k <= j of dA_k,   dP_j = dA_j - slope_h s_j (1 - s_j) C_j,
 *   dq = scale sum_j dP_j k_j,   dk_j += scale dP_j q_i.
 * tests/test_oracle_c.py pins it against oracle/co_alibi_ref.py (itself pinned by closed
 * forms, brute force and finite differences); the two share no code.
 */
#include "co_alibi_ref.h"

#include <math.h>
#include <stdlib.h>

static int visible(int i, int j, int Skv, int causal) { return j < Skv && (!causal || j <= i); }

/* Per-row forward state: p, sigma, P (normalised weights); returns LSE. */
static double row_forward(int i, int Skv, int D, int causal, double scale, double slope, const double* qi,
                          const double* kh, double* p, double* sig, double* prob) {
  double z = 0.0, m = -INFINITY;
  for (int j = 0; j < Skv; ++j) {
    double dot = 0.0;
    for (int d = 0; d < D; ++d) dot += qi[d] * kh[(size_t)j * D + d];
    p[j] = scale * dot;
    sig[j] = visible(i, j, Skv, causal) ? 1.0 / (1.0 + exp(-p[j])) : 0.0;
  }
  /* a_j = p_j - slope * z_j with z the suffix sum of sigma; kept in prob[] for now */
  for (int j = Skv - 1; j >= 0; --j) {
    z += sig[j];
    prob[j] = p[j] - slope * z;
    if (visible(i, j, Skv, causal) && prob[j] > m) m = prob[j];
  }
  double l = 0.0;
  for (int j = 0; j < Skv; ++j) {
    prob[j] = visible(i, j, Skv, causal) ? exp(prob[j] - m) : 0.0;
    l += prob[j];
  }
  l += 1e-9;
  for (int j = 0; j < Skv; ++j) prob[j] /= l;
  return m + log(l);
}

void co_alibi_ref_forward(int B, int Hq, int Hkv, int Sq, int Skv, int D, int causal, double scale,
                          const double* slopes, const double* q, const double* k, const double* v, double* o,
                          double* lse) {
  const int g = Hq / Hkv;
  double* p = (double*)malloc(sizeof(double) * (size_t)(Skv > 0 ? Skv : 1) * 3);
  double* sig = p + Skv;
  double* prob = sig + Skv;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const double* kh = k + ((size_t)b * Hkv + h / g) * Skv * D;
      const double* vh = v + ((size_t)b * Hkv + h / g) * Skv * D;
      for (int i = 0; i < Sq; ++i) {
        const size_t row = ((size_t)b * Hq + h) * Sq + i;
        lse[row] = row_forward(i, Skv, D, causal, scale, slopes[h], q + row * D, kh, p, sig, prob);
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int j = 0; j < Skv; ++j) acc += prob[j] * vh[(size_t)j * D + d];
          o[row * D + d] = acc;
        }
      }
    }
  free(p);
}

void co_alibi_ref_backward(int B, int Hq, int Hkv, int Sq, int Skv, int D, int causal, double scale,
                           const double* slopes, const double* q, const double* k, const double* v,
                           const double* dout, double* dq, double* dk, double* dv) {
  const int g = Hq / Hkv;
  const size_t kv_elems = (size_t)B * Hkv * Skv * D;
  for (size_t e = 0; e < kv_elems; ++e) dk[e] = dv[e] = 0.0;
  double* p = (double*)malloc(sizeof(double) * (size_t)(Skv > 0 ? Skv : 1) * 4);
  double* sig = p + Skv;
  double* prob = sig + Skv;
  double* dpr = prob + Skv;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const size_t kvo = ((size_t)b * Hkv + h / g) * Skv * D;
      const double *kh = k + kvo, *vh = v + kvo;
      for (int i = 0; i < Sq; ++i) {
        const size_t row = ((size_t)b * Hq + h) * Sq + i;
        const double* qi = q + row * D;
        const double* doi = dout + row * D;
        row_forward(i, Skv, D, causal, scale, slopes[h], qi, kh, p, sig, prob);
        double dsum = 0.0;
        for (int j = 0; j < Skv; ++j) {
          double ds = 0.0;
          for (int d = 0; d < D; ++d) {
            ds += doi[d] * vh[(size_t)j * D + d];
            dv[kvo + (size_t)j * D + d] += prob[j] * doi[d];
          }
          dpr[j] = ds; /* dS_j for now */
          dsum += ds * prob[j];
        }
        double c = 0.0;
        for (int j = 0; j < Skv; ++j) {
          const double da = visible(i, j, Skv, causal) ? prob[j] * (dpr[j] - dsum) : 0.0;
          c += da;
          dpr[j] = visible(i, j, Skv, causal) ? da - slopes[h] * sig[j] * (1.0 - sig[j]) * c : 0.0;
        }
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int j = 0; j < Skv; ++j) acc += dpr[j] * kh[(size_t)j * D + d];
          dq[row * D + d] = scale * acc;
        }
        for (int j = 0; j < Skv; ++j)
          for (int d = 0; d < D; ++d) dk[kvo + (size_t)j * D + d] += scale * dpr[j] * qi[d];
      }
    }
  free(p);
}
