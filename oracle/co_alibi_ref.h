/*
 * co_alibi_ref.h - plain-C restatement of Co-ALiBi attention, TEST INFRASTRUCTURE ONLY.
 *
 * Double precision, explicit loops, for tiny shapes.  Only tests/ link it (the C-ABI check
 * program and the cross-check against oracle/co_alibi_ref.py); the product never does.
 *
 * Layout as include/co_alibi.h: q, o, dout, dq are (B, Hq, Sq, D); k, v, dk, dv are
 * (B, Hkv, Skv, D); lse is (B, Hq, Sq); query head h reads key/value head h / (Hq / Hkv).
 * slopes holds Hq penalty slopes.  Causal masking is top-left (key j visible to row i iff
 * j <= i); non-causal masks nothing.
 */
#ifndef CO_ALIBI_REF_H
#define CO_ALIBI_REF_H

#ifdef __cplusplus
extern "C" {
#endif

/* O and LSE (natural log, m + log(l + 1e-9)). */
void co_alibi_ref_forward(int B, int Hq, int Hkv, int Sq, int Skv, int D, int causal, double scale,
                          const double* slopes, const double* q, const double* k, const double* v, double* o,
                          double* lse);

/* dq, dk, dv for upstream gradient dout; dk / dv are summed over each query-head group. */
void co_alibi_ref_backward(int B, int Hq, int Hkv, int Sq, int Skv, int D, int causal, double scale,
                           const double* slopes, const double* q, const double* k, const double* v,
                           const double* dout, double* dq, double* dk, double* dv);

#ifdef __cplusplus
}
#endif

#endif /* CO_ALIBI_REF_H */
