// Co-ALiBi backward on gfx950.
//
// Semantics follow the reference backward (model.py:49-76 with the per-head
// slope as in co_alibi_attn/benchmark_bwd_pass.py:89-91 and the kernel
// co_alibi_attn/co_alibi_bwd_kernel.py:108-146):
//   s_ij  = exp(a_ij - LSE_i)                     (recomputed; a as in the forward)
//   dV_j  = sum_i s_ij dO_i
//   dS_ij = dO_i . v_j
//   D_i   = dO_i . O_i
//   dA_ij = s_ij (dS_ij - D_i)
//   C_ij  = sum_{k <= j} dA_ik                     (inclusive prefix over keys)
//   dP_ij = dA_ij - slope_h * sigma_ij (1 - sigma_ij) C_ij
//   dQ_i  = sm_scale sum_j dP_ij k_j,  dK_j = sm_scale sum_i dP_ij q_i
// For grouped-query attention dK/dV of a key head sum over its query heads.
//
// C and z couple every key of a row, so the backward runs in two passes that
// need no atomics and no per-query-block partial buffers:
//   pass 1 (query-major, keys left to right): S^T, dS^T, dP, dQ^T += K^T dP^T.
//     It writes D_i and cb[i][J] = sum over keys k < 32J of dA_ik.
//   pass 2 (key-major, one work-group per 128 keys of a key head): for every
//     query head of the group and every query tile, S, dS, dP from the forward's
//     zb and pass 1's cb, then dV^T += dO^T s and dK^T += Q^T dP.
// z inside a 32-key block is zb[i][J] minus the exclusive prefix of sigma in
// the block, so no long running sum is ever subtracted from.
#include "coalibi_common.h"
#include "coalibi_kernels.h"

namespace coalibi {

namespace {

constexpr int kBM = 128;  // pass 1: query rows per work-group
constexpr int kBN = 64;   // pass 1: keys per tile
constexpr int kBK = 128;  // pass 2: keys per work-group (32 per wavefront)
constexpr int kBQ = 64;   // pass 2: query rows per tile

template <typename T, int D>
struct BwdCfg {
  static constexpr int CH = 16 / sizeof(T);
  static constexpr int LDR = D + CH;    // row-major tile stride (elements)
  static constexpr int LDT = 64 + CH;   // transposed tile stride (64-row tiles)
  static constexpr int KS = D / 16;
  static constexpr int DT = D / 32;
};

template <bool MASKED, bool CAUSAL>
__device__ __forceinline__ bool pair_ok(int key, int row, int Skv, int Sq) {
  if (!MASKED) return true;
  return key < Skv && row < Sq && (!CAUSAL || key <= row);
}

// ---------------------------------------------------------------------------
// Pass 1: dQ, D, cb.  Layout as in the forward: per wavefront 32 query rows,
// register r of 32-key subtile st of lane (col, hh) <-> key k0 + st*32 + hh*16 + r.
template <typename T, int D, bool CAUSAL, bool MASKED>
__device__ __forceinline__ void dq_tile(const T* __restrict__ sK, const T* __restrict__ sV,
                                        const T* __restrict__ sKt,
                                        const typename Mfma<T>::vec8 (&qf)[BwdCfg<T, D>::KS],
                                        const typename Mfma<T>::vec8 (&dof)[BwdCfg<T, D>::KS],
                                        f32x16 (&acc)[BwdCfg<T, D>::DT], float& crun, float& cb0,
                                        float& cb1, float zb0, float zb1, float lse2, float dsum,
                                        int k0, int row, int col, int hh, int Skv, int Sq, float sc2,
                                        float lam, float lam2) {
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;

  f32x16 sacc[2], dacc[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    sacc[st] = f32x16{};
    dacc[st] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      sacc[st] = M::k16(ld_vec8(sK + (st * 32 + col) * C::LDR + ks * 16 + hh * 8), qf[ks], sacc[st]);
      dacc[st] = M::k16(ld_vec8(sV + (st * 32 + col) * C::LDR + ks * 16 + hh * 8), dof[ks], dacc[st]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  float sg[2][16];
  float tot[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float tv = sacc[st][r] * sc2;
      float s = sigmoid_log2(tv);
      if (MASKED) s = pair_ok<MASKED, CAUSAL>(k0 + st * 32 + hh * 16 + r, row, Skv, Sq) ? s : 0.f;
      sacc[st][r] = tv;
      sg[st][r] = s;
      sum += s;
    }
    tot[st] = sum;
  }
  // z = zb[block] - (exclusive prefix of sigma inside the 32-key block).
  const float oth0 = other_half(tot[0]), oth1 = other_half(tot[1]);
  const float zbase[2] = {zb0 - (hh ? oth0 : 0.f), zb1 - (hh ? oth1 : 0.f)};

  float atot[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    float pre = 0.f, sum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float z = zbase[st] - pre;
      pre += sg[st][r];
      float s = fast_exp2(sacc[st][r] - lam2 * z - lse2);
      if (MASKED) s = pair_ok<MASKED, CAUSAL>(k0 + st * 32 + hh * 16 + r, row, Skv, Sq) ? s : 0.f;
      const float da = s * (dacc[st][r] - dsum);
      dacc[st][r] = da;
      sum += da;
    }
    atot[st] = sum;
  }
  // Inclusive prefix of dA over keys, carried across blocks in crun.
  const float ao0 = other_half(atot[0]), ao1 = other_half(atot[1]);
  const float A00 = hh ? ao0 : atot[0], A01 = hh ? atot[0] : ao0;
  const float A10 = hh ? ao1 : atot[1], A11 = hh ? atot[1] : ao1;
  cb0 = crun;
  cb1 = (cb0 + A00) + A01;
  crun = (cb1 + A10) + A11;
  const float cbase[2] = {cb0 + (hh ? A00 : 0.f), cb1 + (hh ? A10 : 0.f)};

  typename M::vec8 pb[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    float c = cbase[st];
#pragma unroll
    for (int mh = 0; mh < 2; ++mh) {
      f32x8 pv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = mh * 8 + e;
        const float da = dacc[st][r];
        c += da;
        const float sgv = sg[st][r];
        float dp = da - lam * (sgv - sgv * sgv) * c;
        if (MASKED) dp = pair_ok<MASKED, CAUSAL>(k0 + st * 32 + hh * 16 + r, row, Skv, Sq) ? dp : 0.f;
        pv[e] = dp;
      }
      pb[st][mh] = M::pack(pv);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // dQ^T[d][q] += K^T[d][key] dP^T[key][q]
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int mh = 0; mh < 2; ++mh)
        acc[dt] = M::k16(ld_vec8(sKt + (dt * 32 + col) * C::LDT + st * 32 + hh * 16 + mh * 8),
                         pb[st][mh], acc[dt]);
    }
  }
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void coalibi_bwd_dq_kernel(BwdArgs args) {
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  using Tile = TileLoader<T, D, kBN>;
  __shared__ __align__(16) T sK[kBN * C::LDR];
  __shared__ __align__(16) T sV[kBN * C::LDR];
  __shared__ __align__(16) T sKt[D * C::LDT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int Sq = args.Sq, Skv = args.Skv;
  const int nQB = (Sq + kBM - 1) / kBM;
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = wid / nQB;
  const int qb = nQB - 1 - (wid - bh * nQB);
  const int b = bh / args.Hq, hq = bh - b * args.Hq;
  const int hkv = hq / (args.Hq / args.Hkv);
  const size_t qoff = (size_t)bh * Sq * D;
  const size_t kvoff = ((size_t)b * args.Hkv + hkv) * (size_t)Skv * D;
  const T* __restrict__ Kp = static_cast<const T*>(args.k) + kvoff;
  const T* __restrict__ Vp = static_cast<const T*>(args.v) + kvoff;
  const float lam = args.slopes[hq];
  const float lam2 = lam * kLog2e;

  const int q0 = qb * kBM;
  const int wrow0 = q0 + wave * 32;
  const int row = wrow0 + col;
  const bool row_ok = row < Sq;

  vec8 qf[C::KS], dof[C::KS];
  float dpart = 0.f;
  {
    const T* __restrict__ Qr = static_cast<const T*>(args.q) + qoff + (size_t)row * D;
    const T* __restrict__ dOr = static_cast<const T*>(args.dout) + qoff + (size_t)row * D;
    const T* __restrict__ Or = static_cast<const T*>(args.o) + qoff + (size_t)row * D;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const int c0 = ks * 16 + hh * 8;
      qf[ks] = row_ok ? ld_vec8(Qr + c0) : zero_vec8<T>();
      dof[ks] = row_ok ? ld_vec8(dOr + c0) : zero_vec8<T>();
      const vec8 of = row_ok ? ld_vec8(Or + c0) : zero_vec8<T>();
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += (float)dof[ks][e] * (float)of[e];
    }
  }
  const float dsum = dpart + other_half(dpart);
  const float lse2 = row_ok ? args.lse[(size_t)bh * Sq + row] * kLog2e : 0.f;
  if (hh == 0 && row_ok) args.dsum[(size_t)bh * Sq + row] = dsum;

  const int last_key = CAUSAL ? min(q0 + kBM - 1, Skv - 1) : Skv - 1;
  const int nkt = last_key / kBN + 1;

  Tile kregs, vregs;
  kregs.load(Kp, 0, Skv, tid);
  vregs.load(Vp, 0, Skv, tid);

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  float crun = 0.f;
  const float* __restrict__ zb_row = args.zb + (size_t)bh * args.nZB * Sq + row;
  float* __restrict__ cb_row = args.cb + (size_t)bh * args.nZB * Sq + row;

  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();
    kregs.store_rows(sK, C::LDR, tid);
    kregs.store_cols(sKt, C::LDT, tid);
    vregs.store_rows(sV, C::LDR, tid);
    __syncthreads();
    if (kt + 1 < nkt) {
      kregs.load(Kp, (kt + 1) * kBN, Skv, tid);
      vregs.load(Vp, (kt + 1) * kBN, Skv, tid);
    }
    const int k0 = kt * kBN;
    if (CAUSAL && k0 > wrow0 + 31) continue;  // every key of the tile is above this wavefront's rows
    const bool has2 = k0 + 32 < Skv;          // second 32-key block exists
    const float zb0 = row_ok ? zb_row[(size_t)(2 * kt) * Sq] : 0.f;
    const float zb1 = (row_ok && has2) ? zb_row[(size_t)(2 * kt + 1) * Sq] : 0.f;
    const bool masked = (CAUSAL && k0 + kBN - 1 > wrow0) || (k0 + kBN > Skv) || (wrow0 + 32 > Sq);
    float cb0, cb1;
    if (masked)
      dq_tile<T, D, CAUSAL, true>(sK, sV, sKt, qf, dof, acc, crun, cb0, cb1, zb0, zb1, lse2, dsum, k0,
                                  row, col, hh, Skv, Sq, args.sc2, lam, lam2);
    else
      dq_tile<T, D, CAUSAL, false>(sK, sV, sKt, qf, dof, acc, crun, cb0, cb1, zb0, zb1, lse2, dsum, k0,
                                   row, col, hh, Skv, Sq, args.sc2, lam, lam2);
    if (hh == 0 && row_ok) {
      cb_row[(size_t)(2 * kt) * Sq] = cb0;
      if (has2) cb_row[(size_t)(2 * kt + 1) * Sq] = cb1;
    }
  }

  if (row_ok) {
    T* __restrict__ dQr = static_cast<T*>(args.dq) + qoff + (size_t)row * D;
    using vec4 = typename VecOf<T, 4>::type;
    const float sc = args.sm_scale;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v4 = {acc[dt][g * 4 + 0] * sc, acc[dt][g * 4 + 1] * sc, acc[dt][g * 4 + 2] * sc,
                    acc[dt][g * 4 + 3] * sc};
        *reinterpret_cast<vec4*>(dQr + dt * 32 + g * 8 + hh * 4) = __builtin_convertvector(v4, vec4);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 2: dK, dV.  Per wavefront 32 keys (lanes, col = key); accumulator rows
// are queries: register r of query subtile sq of lane (col, hh) <-> query row
// q0 + sq*32 + hh*16 + r.  Key-axis scans run across the 32 lanes of a half.
template <typename T, int D, bool CAUSAL, bool MASKED>
__device__ __forceinline__ void dkdv_tile(const T* __restrict__ sQ, const T* __restrict__ sdO,
                                          const T* __restrict__ sQt, const T* __restrict__ sdOt,
                                          const float* __restrict__ sLse2,
                                          const float* __restrict__ sDsum,
                                          const float* __restrict__ sZb, const float* __restrict__ sCb,
                                          const typename Mfma<T>::vec8 (&kf)[BwdCfg<T, D>::KS],
                                          const typename Mfma<T>::vec8 (&vf)[BwdCfg<T, D>::KS],
                                          f32x16 (&dk)[BwdCfg<T, D>::DT],
                                          f32x16 (&dv)[BwdCfg<T, D>::DT], int sq, int qs0, int key,
                                          int col, int hh, int Skv, int Sq, float sc2, float lam,
                                          float lam2) {
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;

  f32x16 sacc = f32x16{}, dacc = f32x16{};
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    sacc = M::k16(ld_vec8(sQ + (sq * 32 + col) * C::LDR + ks * 16 + hh * 8), kf[ks], sacc);
    dacc = M::k16(ld_vec8(sdO + (sq * 32 + col) * C::LDR + ks * 16 + hh * 8), vf[ks], dacc);
  }
  __builtin_amdgcn_sched_barrier(0);

  const int ql0 = sq * 32 + hh * 16;  // tile-local query of register 0
  typename M::vec8 sb[2], pb[2];
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    f32x8 sv, pv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = mh * 8 + e;
      const int ql = ql0 + r;
      const bool ok = pair_ok<MASKED, CAUSAL>(key, qs0 + hh * 16 + r, Skv, Sq);
      const float tv = sacc[r] * sc2;
      float sg = sigmoid_log2(tv);
      if (MASKED) sg = ok ? sg : 0.f;
      const float pin = half_wave_prefix(sg);
      const float z = sZb[ql] - pin + sg;
      float s = fast_exp2(tv - lam2 * z - sLse2[ql]);
      if (MASKED) s = ok ? s : 0.f;
      const float da = s * (dacc[r] - sDsum[ql]);
      const float c = sCb[ql] + half_wave_prefix(da);
      float dp = da - lam * (sg - sg * sg) * c;
      if (MASKED) dp = ok ? dp : 0.f;
      sv[e] = s;
      pv[e] = dp;
    }
    sb[mh] = M::pack(sv);
    pb[mh] = M::pack(pv);
  }
  __builtin_amdgcn_sched_barrier(0);
  // dV^T[d][key] += dO^T[d][q] s[q][key];  dK^T[d][key] += Q^T[d][q] dP[q][key]
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
    for (int mh = 0; mh < 2; ++mh) {
      const int off = (dt * 32 + col) * C::LDT + sq * 32 + hh * 16 + mh * 8;
      dv[dt] = M::k16(ld_vec8(sdOt + off), sb[mh], dv[dt]);
      dk[dt] = M::k16(ld_vec8(sQt + off), pb[mh], dk[dt]);
    }
  }
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void coalibi_bwd_dkdv_kernel(BwdArgs args) {
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  using Tile = TileLoader<T, D, kBQ>;
  __shared__ __align__(16) T sQ[kBQ * C::LDR];
  __shared__ __align__(16) T sdO[kBQ * C::LDR];
  __shared__ __align__(16) T sQt[D * C::LDT];
  __shared__ __align__(16) T sdOt[D * C::LDT];
  __shared__ __align__(16) float sLse2[kBQ];
  __shared__ __align__(16) float sDsum[kBQ];
  __shared__ __align__(16) float sZb[4][kBQ];
  __shared__ __align__(16) float sCb[4][kBQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int Sq = args.Sq, Skv = args.Skv;
  const int nKB = (Skv + kBK - 1) / kBK;
  const int wid = xcd_remap(blockIdx.x, gridDim.x);
  const int bhk = wid / nKB;               // b * Hkv + hkv
  const int kb = wid - bhk * nKB;          // small kb = most query rows first
  const int b = bhk / args.Hkv, hkv = bhk - b * args.Hkv;
  const int group = args.Hq / args.Hkv;
  const size_t kvoff = (size_t)bhk * Skv * D;
  const int kw0 = kb * kBK + wave * 32;    // first key of this wavefront
  const int key = kw0 + col;

  vec8 kf[C::KS], vf[C::KS];
  {
    const bool key_ok = key < Skv;
    const T* __restrict__ Kr = static_cast<const T*>(args.k) + kvoff + (size_t)key * D;
    const T* __restrict__ Vr = static_cast<const T*>(args.v) + kvoff + (size_t)key * D;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      kf[ks] = key_ok ? ld_vec8(Kr + ks * 16 + hh * 8) : zero_vec8<T>();
      vf[ks] = key_ok ? ld_vec8(Vr + ks * 16 + hh * 8) : zero_vec8<T>();
    }
  }

  f32x16 dk[C::DT], dv[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }

  const int nQT = (Sq + kBQ - 1) / kBQ;
  const int qt0 = CAUSAL ? (kb * kBK) / kBQ : 0;
  Tile qregs, doregs;
  for (int gi = 0; gi < group; ++gi) {
    const int hq = hkv * group + gi;
    const int bh = b * args.Hq + hq;
    const float lam = args.slopes[hq];
    const float lam2 = lam * kLog2e;
    const size_t qoff = (size_t)bh * Sq * D;
    const T* __restrict__ Qp = static_cast<const T*>(args.q) + qoff;
    const T* __restrict__ dOp = static_cast<const T*>(args.dout) + qoff;
    const float* __restrict__ lse = args.lse + (size_t)bh * Sq;
    const float* __restrict__ dsum = args.dsum + (size_t)bh * Sq;
    const float* __restrict__ zb = args.zb + (size_t)bh * args.nZB * Sq;
    const float* __restrict__ cb = args.cb + (size_t)bh * args.nZB * Sq;
    for (int qt = qt0; qt < nQT; ++qt) {
      const int q0 = qt * kBQ;
      qregs.load(Qp, q0, Sq, tid);
      doregs.load(dOp, q0, Sq, tid);
      __syncthreads();
      qregs.store_rows(sQ, C::LDR, tid);
      qregs.store_cols(sQt, C::LDT, tid);
      doregs.store_rows(sdO, C::LDR, tid);
      doregs.store_cols(sdOt, C::LDT, tid);
      {
        // Per-row statistics: tid < 64 -> lse and D, 64..255 -> zb / cb of the wavefronts.
        const int rl = tid & 63;
        const int q = q0 + rl;
        const bool ok = q < Sq;
        if (tid < 64) {
          sLse2[rl] = ok ? lse[q] * kLog2e : 0.f;
          sDsum[rl] = ok ? dsum[q] : 0.f;
        }
        const int w = tid >> 6;  // zb/cb for wavefront w (its 32-key block)
        const int jb = kb * (kBK / 32) + w;
        const bool jok = ok && jb < args.nZB;
        sZb[w][rl] = jok ? zb[(size_t)jb * Sq + q] : 0.f;
        sCb[w][rl] = jok ? cb[(size_t)jb * Sq + q] : 0.f;
      }
      __syncthreads();
      if (kw0 < Skv) {
#pragma unroll
        for (int sq = 0; sq < 2; ++sq) {
          const int qs0 = q0 + sq * 32;
          if (CAUSAL && qs0 + 31 < kw0) continue;  // every row of the subtile precedes the keys
          const bool masked = (CAUSAL && qs0 < kw0 + 31) || (qs0 + 32 > Sq) || (kw0 + 32 > Skv);
          if (masked)
            dkdv_tile<T, D, CAUSAL, true>(sQ, sdO, sQt, sdOt, sLse2, sDsum, sZb[wave], sCb[wave], kf, vf,
                                          dk, dv, sq, qs0, key, col, hh, Skv, Sq, args.sc2, lam, lam2);
          else
            dkdv_tile<T, D, CAUSAL, false>(sQ, sdO, sQt, sdOt, sLse2, sDsum, sZb[wave], sCb[wave], kf,
                                           vf, dk, dv, sq, qs0, key, col, hh, Skv, Sq, args.sc2, lam,
                                           lam2);
        }
      }
      __syncthreads();
    }
  }

  if (key < Skv) {
    using vec4 = typename VecOf<T, 4>::type;
    T* __restrict__ dKr = static_cast<T*>(args.dk) + kvoff + (size_t)key * D;
    T* __restrict__ dVr = static_cast<T*>(args.dv) + kvoff + (size_t)key * D;
    const float sc = args.sm_scale;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = dt * 32 + g * 8 + hh * 4;
        f32x4 k4 = {dk[dt][g * 4 + 0] * sc, dk[dt][g * 4 + 1] * sc, dk[dt][g * 4 + 2] * sc,
                    dk[dt][g * 4 + 3] * sc};
        f32x4 v4 = {dv[dt][g * 4 + 0], dv[dt][g * 4 + 1], dv[dt][g * 4 + 2], dv[dt][g * 4 + 3]};
        *reinterpret_cast<vec4*>(dKr + c0) = __builtin_convertvector(k4, vec4);
        *reinterpret_cast<vec4*>(dVr + c0) = __builtin_convertvector(v4, vec4);
      }
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwd(const BwdArgs& a, int stages, hipStream_t stream) {
  if (stages & 1) {
    const int nQB = (a.Sq + kBM - 1) / kBM;
    hipLaunchKernelGGL((coalibi_bwd_dq_kernel<T, D, CAUSAL>), dim3(nQB * a.B * a.Hq), dim3(256), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & 2) {
    const int nKB = (a.Skv + kBK - 1) / kBK;
    hipLaunchKernelGGL((coalibi_bwd_dkdv_kernel<T, D, CAUSAL>), dim3(nKB * a.B * a.Hkv), dim3(256), 0, stream,
                       a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

#define COALIBI_INST_BWD(T, D)                                           \
  template hipError_t launch_bwd<T, D, true>(const BwdArgs&, int, hipStream_t); \
  template hipError_t launch_bwd<T, D, false>(const BwdArgs&, int, hipStream_t);

COALIBI_INST_BWD(_Float16, 64)
COALIBI_INST_BWD(_Float16, 128)
COALIBI_INST_BWD(__bf16, 64)
COALIBI_INST_BWD(__bf16, 128)
COALIBI_INST_BWD(float, 64)
COALIBI_INST_BWD(float, 128)

}  // namespace coalibi
