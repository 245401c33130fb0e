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
//   pass 1 (query-major, keys left to right from the forward's first processed key):
//     S^T, dS^T, dP, dQ^T += K^T dP^T.  C is the running prefix carry.  z at each 32-key
//     block start is rebuilt from the row's sigmoid total R (saved by the forward, O(S)):
//     z = R minus the sigma totals of the blocks already passed, in fp64.  Each block total
//     is bitwise the one the forward added into R (the same sigmoids, the same order), so z
//     is exact up to its final rounding however large R is, and equal wherever the forward
//     stopped (with or without the tail skip).  Pass 1 writes D_i and, for the recompute
//     path, zb[J][i] (z at the block start) and cb[J][i] (sum of dA over keys before it)
//     into the backward's workspace; for the score-store path, the records.
//   pass 2 (key-major, one work-group per block of keys of a key head): for every
//     query head of the group and every query tile, dV^T += dO^T s and dK^T += Q^T dP,
//     from the score store, or recomputing S^T, dS^T and dP from zb and cb.  Recompute
//     path, fp16/bf16: 64 keys per work-group, a wavefront pair per 32-key group that
//     splits the query tile for S^T/dS^T/dP and the head dim for dV/dK; fp32: 128 keys,
//     one wavefront per 32-key group.
// Both passes hold keys on the accumulator rows (each lane: 16 consecutive keys
// of one query), so both key scans stay in registers.  z inside a 32-key block
// is zb[i][J] minus the exclusive prefix of sigma in the block.
// Operands whose reduction runs over LDS rows (K^T in pass 1; Q^T, dO^T, s, dP
// in pass 2) are read with ds_read_b64_tr_b16 from row-major tiles; the fp32
// validation mode stores transposed copies instead.
#include <type_traits>

#include "coalibi_common.h"
#include "coalibi_kernels.h"

namespace coalibi {

namespace {

constexpr int kBM = 128;  // pass 1: query rows per work-group (32 per wavefront)
constexpr int kBN = 32;   // pass 1: keys per tile
constexpr int kBK = 128;  // pass 2: keys per work-group (32 per wavefront)
// pass 2: query rows per tile (32 in the fp32 validation mode, which also keeps
// transposed copies of the tiles in LDS)
template <typename T>
constexpr int kBQ = sizeof(T) == 4 ? 32 : 64;

template <typename T, int D>
struct BwdCfg {
  static constexpr bool kTr = sizeof(T) == 2;
  static constexpr int CH = 16 / sizeof(T);
  // dQ^T, dK^T and dV^T are produced in 32-row tiles of the head dim: D = 16 runs on a
  // 32-wide head dim whose upper 16 columns are zero in the LDS tiles the products read
  // across d (written once, never loaded over).
  static constexpr int DP = D < 32 ? 32 : D;
  static constexpr int LDR = DP + 2 * CH;  // row-major tile stride (b128 row reads and transpose reads)
  static constexpr int KS = D / 16;
  static constexpr int DT = DP / 32;
  static constexpr int LDT1 = kBN + CH;   // fp32 pass 1: K^T tile stride
  static constexpr int LDT2 = kBQ<T> + CH;  // fp32 pass 2: Q^T / dO^T tile stride
  static constexpr int LDSP = kTr ? 32 + 2 * CH : 32 + CH;  // per-wave s / dP scratch stride
};

__device__ __forceinline__ bool pair_ok(int key, int row, int Skv, int Sq, bool causal) {
  return key < Skv && row < Sq && (!causal || key <= row);
}

// Elementwise core shared by both passes for one 32-key x 32-query tile held as
// S^T (lane (col, hh): query q, keys hh*16 + r).  Inputs: sacc = q.k (times sc2 gives
// log2 units; sc2 = 1 when an operand carries the scale), dacc = dO.v - D (the dS
// accumulator starts at -D = -dO.O), zb = sum of sigma over keys >= the block start,
// cb = sum of dA over keys before the block, lse2 = LSE*log2(e).  Outputs the 16
// values of s and dP packed for the next products; returns the block's dA and sigma totals
// in `atot_blk` and `ztot_blk` (the same value in both halves of the wavefront).  C is carried multiplied by the slope (lam*C), which makes
// dP = dA - lam*sigma'*C one fma per key after sigma' = sigma - sigma^2.
template <typename T, bool MASKED, bool CAUSAL>
__device__ __forceinline__ void dp_tile(const f32x16& sacc, f32x16& dacc, float zb, float cb, float lse2,
                                        int key0, int row, int hh, int Skv, int Sq, float sc2, float lam,
                                        float lam2, typename Mfma<T>::vec8 (&sb)[2],
                                        typename Mfma<T>::vec8 (&pb)[2], float& atot_blk, float& ztot_blk) {
  using M = Mfma<T>;
  // Phase 1: sigma, its inclusive suffix over this run folded into ex = t - lam2*suffix, and
  // the run's sigma total, summed from the run's last key down as the forward sums it.
  float sg[16], ex[16];
  float suf = 0.f;
#pragma unroll
  for (int r = 15; r >= 0; --r) {
    const float t = sacc[r] * sc2;
    float s = sigmoid_log2(t);
    if (MASKED) s = pair_ok(key0 + r, row, Skv, Sq, CAUSAL) ? s : 0.f;
    sg[r] = s;
    suf += s;
    ex[r] = fmaf(-lam2, suf, t);
  }
  // z = zb - (sigma of the other half's run if it is left of ours) - exclusive prefix, and the
  // exclusive prefix is the run total minus the inclusive suffix, so
  // log2 of s = t - lam2*z - lse2 = ex - (lam2*(zb - other - total) + lse2).
  const float tot = suf;
  const float oth = other_half(tot);
  ztot_blk = tot + oth;
  const float zbase = (zb - (hh ? oth : 0.f)) - tot;
  const float cst = fmaf(lam2, zbase, lse2);
  float atot = 0.f;
  f32x8 sv[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float s = fast_exp2(ex[r] - cst);
    if (MASKED) s = pair_ok(key0 + r, row, Skv, Sq, CAUSAL) ? s : 0.f;
    const float da = s * dacc[r];
    dacc[r] = da;
    atot += da;
    sv[r >> 3][r & 7] = s;
  }
  sb[0] = M::pack(sv[0]);
  sb[1] = M::pack(sv[1]);
  // lam*C = lam*(cb + (dA of the other half's run if left of ours) + inclusive prefix).
  const float aoth = other_half(atot);
  float c = lam * (cb + (hh ? aoth : 0.f));
  atot_blk = hh ? atot + aoth : aoth + atot;  // same order in both halves
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    f32x8 pv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = mh * 8 + e;
      const float da = dacc[r];
      c = fmaf(lam, da, c);
      const float sgv = sg[r];
      float dp = fmaf(fmaf(sgv, sgv, -sgv), c, da);  // da - sigma'*lam*C
      if (MASKED) dp = pair_ok(key0 + r, row, Skv, Sq, CAUSAL) ? dp : 0.f;
      pv[e] = dp;
    }
    pb[mh] = M::pack(pv);
  }
}

// ---------------------------------------------------------------------------
// Pass 1: dQ, D, and zb / cb (recompute path) or the score store (STORE).  Per wavefront 32
// query rows; register r of lane (col, hh) <-> key k0 + hh*16 + r.
template <typename T, int D, bool CAUSAL, bool STORE>
__global__ __launch_bounds__(256, (sizeof(T) == 4 || D > 128) ? 1 : 2) void coalibi_bwd_dq_kernel(BwdArgs args) {
  using C = BwdCfg<T, D>;
  // K / V tile row stride: 16-bit rows padded by 48 bytes (76 dwords, 12 mod 32), which reads
  // a little faster than the shared 32-byte pad (1-2 %, measured).
  constexpr int LDR1 = C::kTr ? C::DP + 3 * C::CH : C::LDR;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  using Tile = TileLoader<T, D, kBN, !BwdCfg<T, D>::kTr>;
  static_assert(!STORE || C::kTr, "the score store holds 16-bit operands");
  __shared__ __align__(16) T sK[kBN * LDR1];
  __shared__ __align__(16) T sV[kBN * LDR1];
  __shared__ __align__(16) T sKt[C::kTr ? 8 : C::DP * C::LDT1];
  // STORE: per wavefront, s and dS of its 32 x 32 tile as [row][key], to be read back in
  // operand order.
  constexpr int kScLD = 32 + C::CH;
  __shared__ __align__(16) T sSc[STORE ? 4 * 2 * 32 * kScLD : 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int Sq = args.Sq, Skv = args.Skv;
  const int nQB = (Sq + kBM - 1) / kBM;
  // The fixed order rotates the heads over the XCDs when the tail skip made their work differ;
  // with every head's work alike it keeps each head on one XCD, where its row blocks share the
  // K / V tiles in L2 (full work: -4 % at the headline, measured).
  const int flags = args.flags[0];
  const bool sorted = args.row_order != nullptr && (flags & kFlagRowOrder) != 0;
  const WorkItem item = sorted ? table_item(args.row_order, blockIdx.x, args.B * args.Hq, gridDim.x)
                               : lpt_item(blockIdx.x, args.B * args.Hq, (flags & kFlagTailSkip) ? 1 : 1 << 30);
  const int bh = item.head;
  const int qb = nQB - 1 - item.rank;  // rank 0: the longest causal rows
  const int b = bh / args.Hq, hq = bh - b * args.Hq;
  const int hkv = hq / (args.Hq / args.Hkv);
  const size_t qoff = (size_t)bh * Sq * D;
  const size_t kvoff = ((size_t)b * args.Hkv + hkv) * (size_t)Skv * D;
  const T* __restrict__ Kp = static_cast<const T*>(args.k) + kvoff;
  const T* __restrict__ Vp = static_cast<const T*>(args.v) + kvoff;
  const float lam = args.slopes[hq];
  const float lam2 = lam * kLog2e;
  if constexpr (D < C::DP) {  // padding columns of K (read across d by the dQ product) stay zero
    lds_zero(sK, (int)sizeof(sK), tid, 256);
    if constexpr (!C::kTr) lds_zero(sKt, (int)sizeof(sKt), tid, 256);
  }

  const int q0 = qb * kBM;
  const int wrow0 = q0 + wave * 32;
  const int row = wrow0 + col;
  const bool row_ok = row < Sq;

  const float tile_sc2 = sizeof(T) == 2 ? 1.0f : args.sc2;  // Q carries the scale in 16-bit types
  const int last_key = CAUSAL ? min(q0 + kBM - 1, Skv - 1) : Skv - 1;
  const int nkt = last_key / kBN + 1;
  // Keys left of the forward's first processed key are skipped (their dA and dP are below
  // 2^-T of the row's scale, coalibi_kernels.h); the prefix C starts at zero there.  A kstart
  // past the block's last tile leaves no tile to process.
  static_assert(kBM == kSkipRows, "kstart entries are per pass-1 row block");
  const int kt0 = valid_kstart(args.kstart[(size_t)bh * nQB + qb], Skv) / kBN;

  // The reads before the first tile go out together and share one round trip: the Q / dO / O
  // fragments, the lse and the row's sigmoid total through buffer resources over the block's
  // valid rows (rows past Sq read as zero), then the first K / V tile (its address waits only
  // for kstart).
  vec8 qf[C::KS], dof[C::KS], of[C::KS];
  float lse2, zhi, zlo;
  {
    const int rows = min(Sq - q0, kBM);
    const size_t blk = qoff + (size_t)q0 * D;
    const __amdgpu_buffer_rsrc_t qrs = tile_rsrc(static_cast<const T*>(args.q) + blk, rows * D);
    const __amdgpu_buffer_rsrc_t dors = tile_rsrc(static_cast<const T*>(args.dout) + blk, rows * D);
    const __amdgpu_buffer_rsrc_t ors = tile_rsrc(static_cast<const T*>(args.o) + blk, rows * D);
    const int offb = ((wave * 32 + col) * D + hh * 8) * (int)sizeof(T);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const int off = offb + ks * 16 * (int)sizeof(T);
      qf[ks] = buffer_load_vec8<vec8>(qrs, off);
      dof[ks] = buffer_load_vec8<vec8>(dors, off);
      of[ks] = buffer_load_vec8<vec8>(ors, off);
    }
    const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(args.lse + (size_t)bh * Sq + q0, rows);
    lse2 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lrs, (wave * 32 + col) * 4, 0, 0)) * kLog2e;
    const size_t nrows = (size_t)args.B * args.Hq * Sq;
    const __amdgpu_buffer_rsrc_t hrs = tile_rsrc(args.rsum + (size_t)bh * Sq + q0, rows);
    const __amdgpu_buffer_rsrc_t lors = tile_rsrc(args.rsum + nrows + (size_t)bh * Sq + q0, rows);
    zhi = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(hrs, (wave * 32 + col) * 4, 0, 0));
    zlo = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lors, (wave * 32 + col) * 4, 0, 0));
  }
  float dpart = 0.f;
  // fp32 folds dO.O before the tile loads: holding O across them spills.
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += dof[ks][e] * of[ks][e];
  }
  Tile kregs, vregs;
  kregs.load(Kp, kt0 * kBN, Skv, tid);
  vregs.load(Vp, kt0 * kBN, Skv, tid);
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      // Q pre-scaled by sm_scale*log2(e), as in the forward.
      qf[ks] = scale_vec8<T>(qf[ks], args.sc2);
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += (float)dof[ks][e] * (float)of[ks][e];
    }
  }
  const float dsum = dpart + other_half(dpart);
  if (hh == 0 && row_ok) args.dsum[(size_t)bh * Sq + row] = dsum;

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  float crun = 0.f;
  // z at the next block start: R minus the sigma totals of the blocks passed, in fp64.
  double zsum = (double)zhi + (double)zlo;
  float* __restrict__ zb_row = STORE ? nullptr : args.zb + (size_t)bh * args.nZB * Sq + row;
  float* __restrict__ cb_row = STORE ? nullptr : args.cb + (size_t)bh * args.nZB * Sq + row;
  const int nQ32 = (Sq + 31) / 32;

  // The memory counter completes in order and counts stores: a wait for a load also waits for
  // every store issued before it, and where paths meet the compiler waits for the shortest
  // count of any path.  So that the score-store records drain under the next tiles' work:
  //  - the K/V staging uses barriers that wait for LDS only (__syncthreads waits for the stores);
  //  - the K/V loads and the record stores are buffer operations issued on every path, their
  //    ranges covering only what exists (the rest reads as zero or is dropped);
  //  - the tiles that some wavefront skips (causal: the last ones) run in a loop of their own,
  //    so the skip is not a path of the main loop.
  auto tile = [&](int kt, auto tail) __attribute__((always_inline)) {
    lds_barrier();  // every wavefront's reads of the previous tile are done
    kregs.store_rows(sK, LDR1, tid);
    vregs.store_rows(sV, LDR1, tid);
    if constexpr (!C::kTr) kregs.store_cols(sKt, C::LDT1, tid);
    lds_barrier();  // the tile is in LDS
    kregs.load(Kp, (kt + 1) * kBN, Skv, tid);  // past the last tile: zero rows, never used
    vregs.load(Vp, (kt + 1) * kBN, Skv, tid);
    const int k0 = kt * kBN;
    if constexpr (decltype(tail)::value) {
      // Every key of the tile is above this wavefront's rows, and so are the later tiles'.
      if (CAUSAL && k0 > wrow0 + 31) return;
    }
    const bool masked = (CAUSAL && k0 + kBN - 1 > wrow0) || (k0 + kBN > Skv) || (wrow0 + 32 > Sq);

    f32x16 sacc = f32x16{}, dacc;
    // The 16-register start value of the dS accumulator is rebuilt every tile (16 moves):
    // hoisted out of the loop it would hold 16 registers for the whole kernel.
    float ndsum = -dsum;
    asm volatile("" : "+v"(ndsum));
#pragma unroll
    for (int r = 0; r < 16; ++r) dacc[r] = ndsum;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      sacc = M::k16(ld_vec8(sK + col * LDR1 + ks * 16 + hh * 8), qf[ks], sacc);
      dacc = M::k16(ld_vec8(sV + col * LDR1 + ks * 16 + hh * 8), dof[ks], dacc);
    }
    __builtin_amdgcn_sched_barrier(0);
    vec8 sb[2], pb[2];
    float atot, ztot;
    const float zb = (float)zsum;
    if (masked)
      dp_tile<T, true, CAUSAL>(sacc, dacc, zb, crun, lse2, k0 + hh * 16, row, hh, Skv, Sq, tile_sc2, lam, lam2,
                               sb, pb, atot, ztot);
    else
      dp_tile<T, false, CAUSAL>(sacc, dacc, zb, crun, lse2, k0 + hh * 16, row, hh, Skv, Sq, tile_sc2, lam, lam2,
                                sb, pb, atot, ztot);
    if constexpr (!STORE) {
      if (hh == 0 && row_ok) {
        zb_row[(size_t)kt * Sq] = zb;
        cb_row[(size_t)kt * Sq] = crun;
      }
    }
    crun += atot;
    zsum -= (double)ztot;
    __builtin_amdgcn_sched_barrier(0);
    // dQ^T[d][q] += K^T[d][key] dP^T[key][q];  A rows are keys hh*16 + mh*8 + e.
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        vec8 ka;
        if constexpr (C::kTr)
          ka = ld_kmajor<T, true>(sK, LDR1, mh * 8, 16, dt * 32, lane);
        else
          ka = ld_vec8(sKt + (dt * 32 + col) * C::LDT1 + hh * 16 + mh * 8);
        acc[dt] = M::k16(ka, pb[mh], acc[dt]);
      }
    }
    // Score store: after the dQ products, the tile's s and dS go through this wavefront's
    // LDS scratch ([row][key]) and back out in the operand order of pass 2, one 16-byte store
    // per lane and operand (a record is 4 KB written by one wavefront).  Rows past Sq have
    // no record: their stores fall outside an empty range.
    if constexpr (STORE) {
      T* __restrict__ sc = sSc + wave * 2 * 32 * kScLD;
      *reinterpret_cast<vec8*>(sc + col * kScLD + hh * 16) = sb[0];
      *reinterpret_cast<vec8*>(sc + col * kScLD + hh * 16 + 8) = sb[1];
      *reinterpret_cast<vec8*>(sc + (32 + col) * kScLD + hh * 16) = pb[0];
      *reinterpret_cast<vec8*>(sc + (32 + col) * kScLD + hh * 16 + 8) = pb[1];
      // The transpose reads take other lanes' values: keep the compiler from moving them
      // above the writes (LDS operations of one wavefront execute in order).
      asm volatile("" ::: "memory");
      const u32x4* rec = reinterpret_cast<const u32x4*>(
          static_cast<const char*>(args.scores) +
          ((size_t)bh * args.score_head + score_record(kt, wrow0 / 32, nQ32, CAUSAL)) * kScoreRecordBytes);
      const __amdgpu_buffer_rsrc_t rs = tile_rsrc(rec, wrow0 < Sq ? kScoreRecordBytes / 16 : 0);
      // Non-temporal: each record is written once here and read once by pass 2 (about 8 %
      // faster on both passes than write-back caching, measured).
#pragma unroll
      for (int m = 0; m < 4; ++m)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, ld_kmajor<T, false>(sc + (m >> 1) * 32 * kScLD, kScLD, (m & 1) * 16, 8, 0, lane)),
            rs, (m * 64 + lane) * 16, 0, kCachePolicyNt);
    }
  };
  // Tiles that every wavefront of the block processes (causal: keys up to the block's first
  // row), then the rest.
  const int kt_main = CAUSAL ? max(kt0, min(nkt, q0 / kBN + 1)) : nkt;
  for (int kt = kt0; kt < kt_main; ++kt) tile(kt, std::false_type{});
  for (int kt = kt_main; kt < nkt; ++kt) tile(kt, std::true_type{});

  if (row_ok) {
    T* __restrict__ dQr = static_cast<T*>(args.dq) + qoff + (size_t)row * D;
    using vec4 = typename VecOf<T, 4>::type;
    const float sc = args.sm_scale;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (dt * 32 + g * 8 >= D) continue;  // padding rows of dQ^T (D = 16)
        f32x4 v4 = {acc[dt][g * 4 + 0] * sc, acc[dt][g * 4 + 1] * sc, acc[dt][g * 4 + 2] * sc,
                    acc[dt][g * 4 + 3] * sc};
        *reinterpret_cast<vec4*>(dQr + dt * 32 + g * 8 + hh * 4) = __builtin_convertvector(v4, vec4);
      }
    }
  }
}

// Pass 2's rotation of the heads over the XCDs (balanced_item): runs of kLptRotateRanks key
// blocks of a head share an XCD when the tail skip made the heads' work differ; without it
// every key block of a head stays on one XCD, where they share the head's Q / dO tiles in L2
// (full work: pass 2 -3 % at the headline, -6 % with grouped heads, measured).
__device__ __forceinline__ int pass2_rotate(const BwdArgs& args) {
  return (args.flags[0] & kFlagTailSkip) ? kLptRotateRanks : 1 << 30;
}

// ---------------------------------------------------------------------------
// Pass 2, fp32 validation mode: dK, dV.  Per wavefront the 32 keys kw0.. of one
// 32-key block, held as MFMA A operands (row R <-> key kw0 + kRowOfReg(R)) so that
// register r of lane (col, hh) of S^T <-> key kw0 + hh*16 + r, query q0 + sq*32 + col.
// The 16-bit kernel below splits this work over wavefront pairs; fp32 tiles with
// their transposed copies do not fit the LDS that split needs.  At D = 256 the fp32
// transposed copies alone would not fit either: the reduction's Q^T / dO^T operands are
// then read element by element from the row-major tiles (one 4-byte read per element,
// the 32 lanes of a half reading 32 consecutive head-dim columns of one row).
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void coalibi_bwd_dkdv_f32_kernel(BwdArgs args) {
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  constexpr int BQ = kBQ<T>;
  constexpr bool kCols = !C::kTr && D <= 128;  // transposed copies of the Q and dO tiles in LDS
  using Tile = TileLoader<T, D, BQ, kCols>;
  __shared__ __align__(16) T sQ[BQ * C::LDR];
  __shared__ __align__(16) T sdO[BQ * C::LDR];
  __shared__ __align__(16) T sQt[kCols ? C::DP * C::LDT2 : 8];
  __shared__ __align__(16) T sdOt[kCols ? C::DP * C::LDT2 : 8];
  __shared__ __align__(16) T sSP[4][2][32 * C::LDSP];  // per wavefront: s and dP, [q][key] (fp32: [key][q])
  __shared__ __align__(16) float sLse2[BQ];
  __shared__ __align__(16) float sDsum[BQ];
  __shared__ __align__(16) float sZb[4][BQ];
  __shared__ __align__(16) float sCb[4][BQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int Sq = args.Sq, Skv = args.Skv;
  const int nKB = (Skv + kBK - 1) / kBK;
  static_assert(sizeof(sQ) >= 2 * kMaxBalancedHeads * 4, "the head order is built in sQ");
  const WorkItem item = balanced_item(blockIdx.x, args.B, args.Hkv, args.slopes, args.Hq / args.Hkv,
                                      reinterpret_cast<float*>(sQ), reinterpret_cast<int*>(sQ) + kMaxBalancedHeads,
                                      tid, 256, pass2_rotate(args));
  const int bhk = item.head;               // b * Hkv + hkv
  const int kb = item.rank;                // rank 0: key block 0, seen by the most query rows
  const int b = bhk / args.Hkv, hkv = bhk - b * args.Hkv;
  const int group = args.Hq / args.Hkv;
  const size_t kvoff = (size_t)bhk * Skv * D;
  const int kw0 = kb * kBK + wave * 32;    // first key of this wavefront
  const int jblk = kw0 / 32;               // its 32-key block
  const int key0 = kw0 + hh * 16;          // key of register 0 of this lane
  T* __restrict__ sS = sSP[wave][0];
  T* __restrict__ sP = sSP[wave][1];
  if constexpr (D < C::DP) {  // padding columns of Q and dO (read across d by phase B) stay zero
    lds_zero(sQ, (int)sizeof(sQ), tid, 256);
    lds_zero(sdO, (int)sizeof(sdO), tid, 256);
    if constexpr (kCols) {
      lds_zero(sQt, (int)sizeof(sQt), tid, 256);
      lds_zero(sdOt, (int)sizeof(sdOt), tid, 256);
    }
  }

  vec8 ka[C::KS], va[C::KS];
  {
    const int key = kw0 + kRowOfReg(col);
    const bool key_ok = key < Skv;
    const T* __restrict__ Kr = static_cast<const T*>(args.k) + kvoff + (size_t)key * D;
    const T* __restrict__ Vr = static_cast<const T*>(args.v) + kvoff + (size_t)key * D;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      ka[ks] = key_ok ? ld_vec8(Kr + ks * 16 + hh * 8) : zero_vec8<T>();
      // 16-bit types: K pre-scaled by sm_scale*log2(e), so S^T comes out in log2 units.
      if constexpr (sizeof(T) == 2) ka[ks] = scale_vec8<T>(ka[ks], args.sc2);
      va[ks] = key_ok ? ld_vec8(Vr + ks * 16 + hh * 8) : zero_vec8<T>();
    }
  }
  const float tile_sc2 = sizeof(T) == 2 ? 1.0f : args.sc2;

  f32x16 dk[C::DT], dv[C::DT];
  f32x16 ck[sizeof(T) == 4 ? C::DT : 1], cv[sizeof(T) == 4 ? C::DT : 1];  // fp32: the sums' compensations
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
    if constexpr (sizeof(T) == 4) {
      ck[dt] = f32x16{};
      cv[dt] = f32x16{};
    }
  }

  // Work list: (query head gi, query tile qt) pairs, prefetched one ahead.  Query tiles
  // run from the last one down, so the key blocks of a head that run together read
  // the same Q / dO tiles at about the same time (shared through L2).
  const int nSkipQB = (Sq + kSkipRows - 1) / kSkipRows;  // kstart entries per query head
  const int nQT = (Sq + BQ - 1) / BQ;
  const int qt0 = CAUSAL ? min((kb * kBK) / BQ, nQT) : 0;
  const int per_head = nQT - qt0;
  const int nwork = per_head * group;
  Tile qregs, doregs;
  float st_lse = 0.f, st_dsum = 0.f, st_zb = 0.f, st_cb = 0.f;  // per-row statistics for the next tile
  auto prefetch = [&](int w) {
    const int gi = w / per_head, qt = nQT - 1 - (w - gi * per_head);
    const int bh = b * args.Hq + hkv * group + gi;
    const size_t qoff = (size_t)bh * Sq * D;
    const int q0 = qt * BQ;
    qregs.load(static_cast<const T*>(args.q) + qoff, q0, Sq, tid);
    doregs.load(static_cast<const T*>(args.dout) + qoff, q0, Sq, tid);
    const int q = q0 + lane;
    const bool ok = lane < BQ && q < Sq;
    const int jb = kb * (kBK / 32) + wave;  // the 32-key block of wavefront `wave`
    const bool jok = ok && jb < args.nZB;
    st_lse = ok ? args.lse[(size_t)bh * Sq + q] * kLog2e : 0.f;
    st_dsum = ok ? args.dsum[(size_t)bh * Sq + q] : 0.f;
    st_zb = jok ? args.zb[((size_t)bh * args.nZB + jb) * Sq + q] : 0.f;
    st_cb = jok ? args.cb[((size_t)bh * args.nZB + jb) * Sq + q] : 0.f;
  };
  if (nwork > 0) prefetch(0);

  for (int w = 0; w < nwork; ++w) {
    const int gi = w / per_head, qt = nQT - 1 - (w - gi * per_head);
    const int hq = hkv * group + gi;
    const float lam = args.slopes[hq];
    const float lam2 = lam * kLog2e;
    const int q0 = qt * BQ;
    __syncthreads();
    qregs.template store_rows<false>(sQ, C::LDR, tid);
    doregs.template store_rows<false>(sdO, C::LDR, tid);
    if constexpr (kCols) {
      qregs.store_cols(sQt, C::LDT2, tid);
      doregs.store_cols(sdOt, C::LDT2, tid);
    }
    if (lane < BQ) {
      if (wave == 0) {
        sLse2[lane] = st_lse;
        sDsum[lane] = st_dsum;
      }
      sZb[wave][lane] = st_zb;
      sCb[wave][lane] = st_cb;
    }
    __syncthreads();
    if (w + 1 < nwork) prefetch(w + 1);
    if (kw0 >= Skv) continue;
    // This wavefront's 32 keys lie left of the forward's first processed key for the
    // tile's row block (a multiple of 64): skipped, as pass 1 skipped them (no zb written).
    if (kw0 < valid_kstart(args.kstart[(size_t)(b * args.Hq + hq) * nSkipQB + (q0 / kSkipRows)], Skv)) continue;
#pragma unroll
    for (int sq = 0; sq < BQ / 32; ++sq) {
      const int qs0 = q0 + sq * 32;
      if (CAUSAL && qs0 + 31 < kw0) continue;  // every row of the subtile precedes the keys
      const bool masked = (CAUSAL && qs0 < kw0 + 31) || (qs0 + 32 > Sq) || (kw0 + 32 > Skv);
      const int ql = sq * 32 + col;  // tile-local query row of this lane
      const int row = qs0 + col;

      f32x16 sacc = f32x16{}, dacc;
      const float dsum = sDsum[ql];
#pragma unroll
      for (int r = 0; r < 16; ++r) dacc[r] = -dsum;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        sacc = M::k16(ka[ks], ld_vec8(sQ + ql * C::LDR + ks * 16 + hh * 8), sacc);
        dacc = M::k16(va[ks], ld_vec8(sdO + ql * C::LDR + ks * 16 + hh * 8), dacc);
      }
      __builtin_amdgcn_sched_barrier(0);
      vec8 sb[2], pb[2];
      float atot, ztot;
      if (masked)
        dp_tile<T, true, CAUSAL>(sacc, dacc, sZb[wave][ql], sCb[wave][ql], sLse2[ql], key0, row, hh, Skv, Sq,
                                 tile_sc2, lam, lam2, sb, pb, atot, ztot);
      else
        dp_tile<T, false, CAUSAL>(sacc, dacc, sZb[wave][ql], sCb[wave][ql], sLse2[ql], key0, row, hh, Skv, Sq,
                                  tile_sc2, lam, lam2, sb, pb, atot, ztot);
      // s and dP to this wavefront's scratch, then back as operands reduced over queries.
      if constexpr (C::kTr) {
        *reinterpret_cast<vec8*>(sS + col * C::LDSP + hh * 16) = sb[0];
        *reinterpret_cast<vec8*>(sS + col * C::LDSP + hh * 16 + 8) = sb[1];
        *reinterpret_cast<vec8*>(sP + col * C::LDSP + hh * 16) = pb[0];
        *reinterpret_cast<vec8*>(sP + col * C::LDSP + hh * 16 + 8) = pb[1];
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sS[(hh * 16 + r) * C::LDSP + col] = sb[r >> 3][r & 7];
          sP[(hh * 16 + r) * C::LDSP + col] = pb[r >> 3][r & 7];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // dV^T[d][key] += dO^T[d][q] s[q][key];  dK^T[d][key] += Q^T[d][q] dP[q][key]
      // reduction rows (queries) mh*16 + kh*8 + e of the subtile.  The subtile's 32 queries
      // are summed in a fresh accumulator that is then added to the running one: one rounding
      // at the running sum's magnitude per subtile instead of one per product step (in fp32
      // a plain running dK / dV over a long grouped row range drifts by ~1e-4 at |dV| ~ 100).
      vec8 sop[2], pop[2];
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        if constexpr (C::kTr) {
          sop[mh] = ld_kmajor<T, false>(sS, C::LDSP, mh * 16, 8, 0, lane);
          pop[mh] = ld_kmajor<T, false>(sP, C::LDSP, mh * 16, 8, 0, lane);
        } else {
          sop[mh] = ld_vec8(sS + col * C::LDSP + mh * 16 + hh * 8);
          pop[mh] = ld_vec8(sP + col * C::LDSP + mh * 16 + hh * 8);
        }
      }
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        f32x16 tv = f32x16{}, tk = f32x16{};
#pragma unroll
        for (int mh = 0; mh < 2; ++mh) {
          vec8 doa, qa;
          if constexpr (C::kTr) {
            doa = ld_kmajor<T, false>(sdO, C::LDR, sq * 32 + mh * 16, 8, dt * 32, lane);
            qa = ld_kmajor<T, false>(sQ, C::LDR, sq * 32 + mh * 16, 8, dt * 32, lane);
          } else if constexpr (kCols) {
            doa = ld_vec8(sdOt + (dt * 32 + col) * C::LDT2 + sq * 32 + mh * 16 + hh * 8);
            qa = ld_vec8(sQt + (dt * 32 + col) * C::LDT2 + sq * 32 + mh * 16 + hh * 8);
          } else {
            const int r0 = sq * 32 + mh * 16 + hh * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              doa[e] = sdO[(r0 + e) * C::LDR + dt * 32 + col];
              qa[e] = sQ[(r0 + e) * C::LDR + dt * 32 + col];
            }
          }
          tv = M::k16(doa, sop[mh], tv);
          tk = M::k16(qa, pop[mh], tk);
        }
        if constexpr (sizeof(T) == 4) {
          // fp32: compensated (Kahan) running sums, so the running dK / dV stay within a few
          // ulps over any number of subtiles.
          const f32x16 yv = tv - cv[dt], yk = tk - ck[dt];
          const f32x16 sv = dv[dt] + yv, sk = dk[dt] + yk;
          cv[dt] = (sv - dv[dt]) - yv;
          ck[dt] = (sk - dk[dt]) - yk;
          dv[dt] = sv;
          dk[dt] = sk;
        } else {
          dv[dt] += tv;
          dk[dt] += tk;
        }
      }
    }
  }
  (void)jblk;

  const int key = kw0 + col;
  if (key < Skv) {
    using vec4 = typename VecOf<T, 4>::type;
    T* __restrict__ dKr = static_cast<T*>(args.dk) + kvoff + (size_t)key * D;
    T* __restrict__ dVr = static_cast<T*>(args.dv) + kvoff + (size_t)key * D;
    const float sc = args.sm_scale;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (dt * 32 + g * 8 >= D) continue;  // padding rows of dK^T / dV^T (D = 16)
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


// Pass 2 for fp16/bf16: dK, dV with wavefront pairs.  A work-group of 4
// wavefronts owns 64 keys in two key groups kg of 32 and walks query tiles of 64
// rows.  Wavefront (kg, qh) holds K of its key group as MFMA A operands (as
// above; V comes from LDS) and computes S^T, dS^T and then s, dP for query half qh
// of the tile into its key group's LDS buffer.  After a barrier each wavefront of
// the pair reduces over all 64 queries of the tile, but only for its half of the
// head dim:
//   dV^T[d][key] += dO^T[d][q] s[q][key],  dK^T[d][key] += Q^T[d][q] dP[q][key],
// for d in [qh*D/2, qh*D/2 + D/2).  Splitting the accumulators and the score tile
// this way halves the registers of the one-wavefront-per-key-group form, so two
// work-groups share a CU (two wavefronts per SIMD from independent work-groups,
// whose barriers do not align their phases) at no extra elementwise work.  The
// next Q and dO tiles arrive by buffer-to-LDS DMA issued once the current tile is
// no longer read; the other work-group on the CU covers that latency.
// Pass 2's work list for one block of keys of a key head: (query head gi, query tile qt)
// pairs, qt from qt_hi(gi) down to qt0 (the first tile that can see the block).  Tail skip:
// kstart, the first key the forward processed for a 128-row block, is a multiple of 64, so
// for every 64-row tile a 64-key block is processed or skipped as a whole.  qt_hi(gi) is the
// last tile of head gi whose row block processed the keys (found once, in LDS, for up to
// kMaxPairGroup query heads per key head; all tiles otherwise); a tile inside the range whose
// row block skipped them is left out by the caller's own kstart test.
constexpr int kMaxPairGroup = 64;
struct KeyBlockWork {
  int group, nQT, qt0;
  bool ranged;
  const int* qthi;  // LDS, one entry per query head of the group
  __device__ __forceinline__ int qt_hi(int g) const { return ranged ? qthi[g] : nQT - 1; }
  // the first head from g on with a tile in range, or group
  __device__ __forceinline__ int next_head(int g) const {
    while (g < group && qt_hi(g) < qt0) ++g;
    return g;
  }
  __device__ __forceinline__ int count() const {
    int n = 0;
    for (int g = 0; g < group; ++g) n += max(qt_hi(g) - qt0 + 1, 0);
    return n;
  }
};
// Fills qthi for a key block starting at key kwg0 (wavefront w: heads w, w + nwaves, ...);
// the caller synchronises before reading it.  BQ rows per tile, two tiles per kstart entry.
template <int BQ>
__device__ __forceinline__ KeyBlockWork key_block_work(int* qthi, const int* __restrict__ kstart_g, int group,
                                                       int Sq, int Skv, int qt0, int kwg0, int wave, int nwaves,
                                                       int lane) {
  static_assert(BQ * 2 == kSkipRows, "two query tiles per kstart row block");
  const int nQT = (Sq + BQ - 1) / BQ;
  const int nSkipQB = (Sq + kSkipRows - 1) / kSkipRows;
  const bool ranged = group <= kMaxPairGroup;
  if (ranged) {
    for (int g = wave; g < group; g += nwaves) {
      int hi = qt0 - 1;
      for (int rb = lane; rb < nSkipQB; rb += 64)
        if (valid_kstart(kstart_g[(size_t)g * nSkipQB + rb], Skv) <= kwg0) hi = max(hi, min(2 * rb + 1, nQT - 1));
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) hi = max(hi, __shfl_xor(hi, off));
      if (lane == 0) qthi[g] = hi;
    }
  }
  return {group, nQT, qt0, ranged, qthi};
}

constexpr int kPairBK = 64;     // keys per work-group
constexpr int kPairBQ = 64;     // query rows per tile
constexpr int kPairWaves = 4;   // wavefronts per work-group: 2 key groups x 2 query halves
// Two work-groups per CU: 77 KB of LDS and at most 256 VGPRs each.

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(64 * kPairWaves, D > 128 ? 1 : 2) void coalibi_bwd_dkdv_kernel(BwdArgs args) {
  static_assert(sizeof(T) == 2, "the wavefront-pair pass 2 is the 16-bit path");
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  constexpr int BQ = kPairBQ;
  constexpr int NKG = kPairBK / 32;
  constexpr int DH = C::DT / 2;                   // 32-row tiles of d per wavefront
  constexpr int TILE = BQ * C::LDR;               // elements of one padded Q or dO tile
  using Dma = DmaTile<T, D, BQ, C::LDR, kPairWaves, false>;
  constexpr int LDSP = 32 + C::CH;  // s / dP rows: 32 keys + one 16-byte pad
  __shared__ __align__(16) T sQ[1][TILE];   // one buffer: the next tile lands after this one is read
  __shared__ __align__(16) T sdO[1][TILE];
  __shared__ __align__(16) T sV[kPairBK * C::LDR];       // V rows, permuted per 32-key group
  __shared__ __align__(16) T sSP[NKG][2][BQ * LDSP];     // per key group: s and dP, [q][key]
  __shared__ __align__(16) float sLse2[2][BQ];
  __shared__ __align__(16) float sDsum[2][BQ];
  __shared__ __align__(16) float sZb[2][NKG][BQ];
  __shared__ __align__(16) float sCb[2][NKG][BQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int kg = wave >> 1, qh = wave & 1;
  const int Sq = args.Sq, Skv = args.Skv;
  static_assert(sizeof(sSP) >= 2 * kMaxBalancedHeads * 4, "the head order is built in sSP");
  const bool sorted = args.key_order != nullptr && (args.flags[0] & kFlagKeyOrder) != 0;
  const WorkItem item =
      sorted ? table_item(args.key_order, blockIdx.x, args.B * args.Hkv, gridDim.x)
             : balanced_item(blockIdx.x, args.B, args.Hkv, args.slopes, args.Hq / args.Hkv,
                                     reinterpret_cast<float*>(&sSP[0][0][0]),
                                     reinterpret_cast<int*>(&sSP[0][0][0]) + kMaxBalancedHeads, tid, 64 * kPairWaves,
                                     pass2_rotate(args));
  const int bhk = item.head;               // b * Hkv + hkv
  const int kb = item.rank;                // rank 0: key block 0, seen by the most query rows
  const int b = bhk / args.Hkv, hkv = bhk - b * args.Hkv;
  const int group = args.Hq / args.Hkv;
  const size_t kvoff = (size_t)bhk * Skv * D;
  const int kw0 = kb * kPairBK + kg * 32;  // first key of this wavefront's key group
  const int key0 = kw0 + hh * 16;          // key of register 0 of this lane
  const bool keys_ok = kw0 < Skv;
  T* __restrict__ sS = sSP[kg][0];
  T* __restrict__ sP = sSP[kg][1];

  // The work-group's reads before its first tile go out together and share one round
  // trip: K fragments into registers, the V tile by buffer-to-LDS DMA (LDS row R of each
  // 32-row group holds key kRowOfReg(R) of the group, the A-operand order; keys past Skv
  // land as zero) and, below, the forward's kstart rows of the group's heads.
  vec8 ka[C::KS];
  {
    const bool key_ok = kw0 + kRowOfReg(col) < Skv;
    const T* __restrict__ Kr = static_cast<const T*>(args.k) + kvoff + (size_t)(kw0 + kRowOfReg(col)) * D;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) ka[ks] = key_ok ? ld_vec8(Kr + ks * 16 + hh * 8) : zero_vec8<T>();
  }
  {
    using VDma = DmaTile<T, D, kPairBK, C::LDR, kPairWaves, true>;
    static_assert(VDma::LDS_ELEMS == kPairBK * C::LDR, "the V DMA writes exactly the V tile");
    VDma vdma;
    vdma.init(wave, lane);
    vdma.issue(static_cast<const T*>(args.v) + kvoff, kb * kPairBK, Skv, sV, wave);
  }
  const T* __restrict__ sVg = sV + kg * 32 * C::LDR;

  f32x16 dk[DH], dv[DH];
#pragma unroll
  for (int i = 0; i < DH; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }

  Dma dma;  // the Q and dO tiles share the chunk layout
  static_assert(Dma::LDS_ELEMS == TILE, "every DMA writes its whole tile (pad and tail chunks as zero)");
  dma.init(wave, lane);

  // Work list (key_block_work): (query head gi, query tile qt) pairs.
  __shared__ int sQtHi[kMaxPairGroup];
  const int nQT = (Sq + BQ - 1) / BQ;
  const int qt0 = CAUSAL ? min((kb * kPairBK) / BQ, nQT) : 0;
  const int nSkipQB = (Sq + kSkipRows - 1) / kSkipRows;
  const int kwg0 = kb * kPairBK;
  const int* __restrict__ kstart_g = args.kstart + (size_t)(b * args.Hq + hkv * group) * nSkipQB;
  const KeyBlockWork work =
      key_block_work<BQ>(sQtHi, kstart_g, group, Sq, Skv, qt0, kwg0, wave, kPairWaves, lane);
  // K pre-scaled by sm_scale*log2(e), so S^T comes out in log2 units.
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) ka[ks] = scale_vec8<T>(ka[ks], args.sc2);
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's V DMA
  __syncthreads();                // the V tile and sQtHi
  auto qt_hi = [&](int g) { return work.qt_hi(g); };
  auto next_head = [&](int g) { return work.next_head(g); };
  const int nwork = work.count();
  const int jb = kw0 / 32;  // this key group's 32-key block
  auto issue_tile = [&](int gi, int qt, int buf) {
    const size_t qoff = (size_t)(b * args.Hq + hkv * group + gi) * Sq * D;
    dma.issue(static_cast<const T*>(args.q) + qoff, qt * BQ, Sq, sQ[buf], wave);
    dma.issue(static_cast<const T*>(args.dout) + qoff, qt * BQ, Sq, sdO[buf], wave);
  };
  // Per-row statistics of a tile, one value per lane (= tile row) through buffer
  // loads (rows past Sq and blocks past the last read as zero): wavefront 0 loads
  // LSE, wavefront 1 loads D, and the two wavefronts of a key group load its zb and cb.
  float st_a = 0.f, st_b = 0.f;
  auto load_stats = [&](int gi, int qt) {
    const size_t bh = (size_t)b * args.Hq + hkv * group + gi;
    const int q0 = qt * BQ;
    const int rows = min(max(Sq - q0, 0), BQ);
    if (wave < 2) {
      const float* src = (wave == 0 ? args.lse : args.dsum) + bh * Sq + q0;
      st_a = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(src, rows), lane * 4, 0, 0));
    }
    const float* blk = (qh == 0 ? args.zb : args.cb) + (bh * args.nZB + jb) * Sq + q0;
    st_b = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(blk, jb < args.nZB ? rows : 0),
                                                                          lane * 4, 0, 0));
  };
  auto store_stats = [&](int buf) {
    if (wave == 0) sLse2[buf][lane] = st_a * kLog2e;
    if (wave == 1) sDsum[buf][lane] = st_a;
    if (qh == 0) sZb[buf][kg][lane] = st_b;
    else sCb[buf][kg][lane] = st_b;
  };

  // Query tiles run from the last one down: the key blocks of a head that run together
  // then read the same Q / dO tiles at about the same time (shared through L2).
  int gi = next_head(0), qt = gi < group ? qt_hi(gi) : 0;  // current work item; the next one is (gn, qn)
  if (nwork > 0) {
    issue_tile(gi, qt, 0);
    load_stats(gi, qt);
    __builtin_amdgcn_s_waitcnt(0);  // the stats loads have to land before they are stored
    store_stats(0);
  }

  for (int w = 0; w < nwork; ++w) {
    const int buf = w & 1;  // statistics buffer
    const bool wrap = qt == qt0;
    const int gn = wrap ? next_head(gi + 1) : gi;
    const int qn = wrap ? (gn < group ? qt_hi(gn) : 0) : qt - 1;
    const int hq = hkv * group + gi;
    const float lam = args.slopes[hq];
    const float lam2 = lam * kLog2e;
    const int q0 = qt * BQ;
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's DMA of tile w
    __syncthreads();                // every wavefront's DMA of tile w landed
    if (w + 1 < nwork) load_stats(gn, qn);
    const T* __restrict__ tQ = sQ[0];
    const T* __restrict__ tdO = sdO[0];

    // Query half h of the tile meets this key group (some pair is visible) and the
    // forward processed these keys for the tile's row block.
    const bool processed = kwg0 >= valid_kstart(kstart_g[(size_t)gi * nSkipQB + qt / 2], Skv);
    auto half_live = [&](int h) {
      const int qs0 = q0 + h * 32;
      return processed && keys_ok && qs0 < Sq && (!CAUSAL || qs0 + 31 >= kw0);
    };
    if (half_live(qh)) {
      const int qs0 = q0 + qh * 32;
      const bool masked = (CAUSAL && qs0 < kw0 + 31) || (qs0 + 32 > Sq) || (kw0 + 32 > Skv);
      const int ql = qh * 32 + col;  // tile-local query row of this lane
      const int row = qs0 + col;
      f32x16 sacc = f32x16{}, dacc;
      const float dsum = sDsum[buf][ql];
#pragma unroll
      for (int r = 0; r < 16; ++r) dacc[r] = -dsum;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        sacc = M::k16(ka[ks], ld_vec8(tQ + ql * C::LDR + ks * 16 + hh * 8), sacc);
        dacc = M::k16(ld_vec8(sVg + col * C::LDR + ks * 16 + hh * 8), ld_vec8(tdO + ql * C::LDR + ks * 16 + hh * 8),
                      dacc);
      }
      vec8 sb[2], pb[2];
      float atot, ztot;
      if (masked)
        dp_tile<T, true, CAUSAL>(sacc, dacc, sZb[buf][kg][ql], sCb[buf][kg][ql], sLse2[buf][ql], key0, row, hh,
                                 Skv, Sq, 1.0f, lam, lam2, sb, pb, atot, ztot);
      else
        dp_tile<T, false, CAUSAL>(sacc, dacc, sZb[buf][kg][ql], sCb[buf][kg][ql], sLse2[buf][ql], key0, row, hh,
                                  Skv, Sq, 1.0f, lam, lam2, sb, pb, atot, ztot);
      *reinterpret_cast<vec8*>(sS + ql * LDSP + hh * 16) = sb[0];
      *reinterpret_cast<vec8*>(sS + ql * LDSP + hh * 16 + 8) = sb[1];
      *reinterpret_cast<vec8*>(sP + ql * LDSP + hh * 16) = pb[0];
      *reinterpret_cast<vec8*>(sP + ql * LDSP + hh * 16 + 8) = pb[1];
    }
    __syncthreads();
    // Reduce over the live query halves: reduction rows h*32 + mh*16 + kh*8 + e.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (!half_live(h)) continue;
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        const vec8 sop = ld_kmajor<T, false>(sS, LDSP, h * 32 + mh * 16, 8, 0, lane);
        const vec8 pop = ld_kmajor<T, false>(sP, LDSP, h * 32 + mh * 16, 8, 0, lane);
#pragma unroll
        for (int i = 0; i < DH; ++i) {
          const int dt = qh * DH + i;
          const vec8 doa = ld_kmajor<T, false>(tdO, C::LDR, h * 32 + mh * 16, 8, dt * 32, lane);
          const vec8 qa = ld_kmajor<T, false>(tQ, C::LDR, h * 32 + mh * 16, 8, dt * 32, lane);
          dv[i] = M::k16(doa, sop, dv[i]);
          dk[i] = M::k16(qa, pop, dk[i]);
        }
      }
    }
    // Statistics of tile w+1 (loaded during this tile) into the other buffer; that
    // buffer was last read in tile w-1.
    if (w + 1 < nwork) {
      store_stats(buf ^ 1);
      __syncthreads();  // tile w and the score buffers are no longer read
      issue_tile(gn, qn, 0);
    }
    gi = gn;
    qt = qn;
  }

  const int key = kw0 + col;
  if (key < Skv) {
    using vec4 = typename VecOf<T, 4>::type;
    T* __restrict__ dKr = static_cast<T*>(args.dk) + kvoff + (size_t)key * D;
    T* __restrict__ dVr = static_cast<T*>(args.dv) + kvoff + (size_t)key * D;
    const float sc = args.sm_scale;
#pragma unroll
    for (int i = 0; i < DH; ++i) {
      const int dt = qh * DH + i;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = dt * 32 + g * 8 + hh * 4;
        f32x4 k4 = {dk[i][g * 4 + 0] * sc, dk[i][g * 4 + 1] * sc, dk[i][g * 4 + 2] * sc, dk[i][g * 4 + 3] * sc};
        f32x4 v4 = {dv[i][g * 4 + 0], dv[i][g * 4 + 1], dv[i][g * 4 + 2], dv[i][g * 4 + 3]};
        *reinterpret_cast<vec4*>(dKr + c0) = __builtin_convertvector(k4, vec4);
        *reinterpret_cast<vec4*>(dVr + c0) = __builtin_convertvector(v4, vec4);
      }
    }
  }
}

// Pass 2 from the score store (16-bit types, D = 64 or 128): dK and dV of 64 keys per
// work-group, reduced from the s and dS records pass 1 wrote; nothing is recomputed.
//   dV^T[d][key] += dO^T[d][q] s[q][key],  dK^T[d][key] += Q^T[d][q] dS[q][key].
// Wavefront (kg, qh) accumulates key group kg (32 keys) over query half qh of every 64-row
// tile, for the whole head dim; at the end the two halves are added through LDS.  The
// B operands come from the records straight into registers (they are stored in MFMA lane
// order), one tile ahead; the A operands are transpose reads of the Q and dO tiles, which
// arrive by untracked buffer-to-LDS DMA into two buffers, one tile ahead.  One barrier per
// tile: it publishes tile w and frees the buffer of tile w - 1 for tile w + 1.
constexpr int kStoreBK = 64;  // keys per work-group
constexpr int kStoreBQ = 64;  // query rows per tile

// LISTED: the key block's work items fit kStoreProcessedWords (group * query tiles, checked by
// the launcher); they are then listed in LDS once, in walk order, each with its row block's
// processed bit, in place of the per-head bit words and the walk in the loop.
template <typename T, int D, bool CAUSAL, bool LISTED>
__global__ __launch_bounds__(256, 2) void coalibi_bwd_dkdv_store_kernel(BwdArgs args) {
  static_assert(sizeof(T) == 2 && (D == 64 || D == 128), "the score store path is 16-bit, D 64 or 128");
  using C = BwdCfg<T, D>;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  constexpr int BQ = kStoreBQ;
  constexpr int TILE = BQ * C::LDR;
  using Dma = DmaTile<T, D, BQ, C::LDR, 4, false>;
  static_assert(Dma::LDS_ELEMS == TILE, "every DMA writes its whole tile (pad and tail chunks as zero)");
  __shared__ __align__(16) T sQ[2][TILE];
  __shared__ __align__(16) T sdO[2][TILE];
  __shared__ int sQtHi[kMaxPairGroup];
  // Whether the forward processed this key block for row block rb of query head g: bit rb % 32
  // of word g * wph + rb / 32, or with LISTED the work items (kstart copied once, before any
  // untracked DMA: loads after those cannot be proven unclobbered and would go through the
  // vector memory counter, whose waits would also wait for the DMA).
  __shared__ unsigned sProc[kStoreProcessedWords];
  // The end-of-block exchange: 2 key groups x DT*16 accumulators x 64 lanes per half.
  static_assert(2 * C::DT * 16 * 64 * sizeof(float) <= sizeof(sQ), "the exchange fits one tile pair");

  // wave is uniform; readfirstlane lets the DMA slot choice stay scalar.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, hh = lane >> 5;
  const int kg = wave >> 1, qh = wave & 1;
  const int Sq = args.Sq, Skv = args.Skv;
  static_assert(sizeof(sQ[1]) >= 2 * kMaxBalancedHeads * 4, "the head order is built in sQ[1]");
  const bool sorted = args.key_order != nullptr && (args.flags[0] & kFlagKeyOrder) != 0;
  const WorkItem item = sorted ? table_item(args.key_order, blockIdx.x, args.B * args.Hkv, gridDim.x)
                               : balanced_item(blockIdx.x, args.B, args.Hkv, args.slopes, args.Hq / args.Hkv,
                                               reinterpret_cast<float*>(sQ[1]),
                                               reinterpret_cast<int*>(sQ[1]) + kMaxBalancedHeads, tid, 256,
                                               pass2_rotate(args));
  const int bhk = item.head;  // b * Hkv + hkv
  const int kb = item.rank;   // rank 0: key block 0, seen by the most query rows
  const int b = bhk / args.Hkv, hkv = bhk - b * args.Hkv;
  const int group = args.Hq / args.Hkv;
  const size_t kvoff = (size_t)bhk * Skv * D;
  const int kwg0 = kb * kStoreBK;
  const int kw0 = kwg0 + kg * 32;  // first key of this wavefront's key group
  const int jb = kw0 / 32;
  const bool keys_ok = kw0 < Skv;

  const int nQT = (Sq + BQ - 1) / BQ;
  const int qt0 = CAUSAL ? min(kwg0 / BQ, nQT) : 0;
  const int nSkipQB = (Sq + kSkipRows - 1) / kSkipRows;
  const int* __restrict__ kstart_g = args.kstart + (size_t)(b * args.Hq + hkv * group) * nSkipQB;
  const KeyBlockWork work = key_block_work<BQ>(sQtHi, kstart_g, group, Sq, Skv, qt0, kwg0, wave, 4, lane);
  const int wph = (nSkipQB + 63) / 64 * 2;  // words per head (the host checks group * wph fits)
  if constexpr (LISTED) {
    __syncthreads();  // sQtHi
    // Item i of the walk: query head gi, tile qt (from qt_hi(gi) down to qt0), as
    // gi << 16 | qt << 1 | processed.
    for (int i = tid; i < kStoreProcessedWords; i += 256) {
      int gi = 0, base = 0;
      for (; gi < group; ++gi) {
        const int n = max(work.qt_hi(gi) - qt0 + 1, 0);
        if (i < base + n) break;
        base += n;
      }
      if (gi < group) {
        const int qt = work.qt_hi(gi) - (i - base);
        const bool proc = valid_kstart(kstart_g[(size_t)gi * nSkipQB + qt / 2], Skv) <= kwg0;
        sProc[i] = (unsigned)gi << 16 | (unsigned)qt << 1 | (proc ? 1u : 0u);
      }
    }
  } else {
    for (int g = wave; g < group; g += 4) {
      for (int rb0 = 0; rb0 < nSkipQB; rb0 += 64) {
        const int rb = rb0 + lane;
        const unsigned long long m =
            __ballot(rb < nSkipQB && valid_kstart(kstart_g[(size_t)g * nSkipQB + rb], Skv) <= kwg0);
        if (lane == 0) {
          sProc[g * wph + rb0 / 32] = static_cast<unsigned>(m);
          sProc[g * wph + rb0 / 32 + 1] = static_cast<unsigned>(m >> 32);
        }
      }
    }
  }
  __syncthreads();  // sQtHi, sProc; the head-order scratch in sQ[1] is free again
  const int nwork = work.count();
  const int nQ32 = (Sq + 31) / 32;

  Dma dma;
  dma.init(wave, lane);
  // Loop invariants kept in scalar registers: the LDS addresses of the tile buffers, the Q / dO
  // of the group's first query head and the head stride.
  const unsigned lds_q = lds_address(sQ[0]), lds_do = lds_address(sdO[0]);
  const size_t head0 = (size_t)(b * args.Hq + hkv * group) * Sq * D, head_stride = (size_t)Sq * D;
  const T* __restrict__ q_g = static_cast<const T*>(args.q) + head0;
  const T* __restrict__ do_g = static_cast<const T*>(args.dout) + head0;
  auto issue_tile = [&](int gi, int qt, int buf) {
    const size_t qoff = (size_t)gi * head_stride;
    const unsigned lbuf = (unsigned)(buf * TILE * (int)sizeof(T));
    dma.issue_untracked(q_g + qoff, qt * BQ, Sq, lds_q + lbuf, wave);
    dma.issue_untracked(do_g + qoff, qt * BQ, Sq, lds_do + lbuf, wave);
  };
  // A work item: query head gi, query tile qt, and whether the forward processed this key block
  // for the tile's row block.
  struct Item {
    int gi, qt;
    bool proc;
  };
  auto walked = [&](int gi, int qt) {
    const int rb = qt / 2;
    return Item{gi, qt, ((sProc[gi * wph + rb / 32] >> (rb % 32)) & 1u) != 0};
  };
  auto listed = [&](int i) {
    const unsigned e = __builtin_amdgcn_readfirstlane(sProc[i]);
    return Item{(int)(e >> 16), (int)((e >> 1) & 0x7fffu), (e & 1u) != 0};
  };
  // This wavefront's query half of tile qt holds visible pairs of its key group that the
  // forward processed: exactly the records pass 1 wrote.
  auto live = [&](const Item& it) {
    const int qs0 = it.qt * BQ + qh * 32;
    return it.proc && keys_ok && qs0 < Sq && (!CAUSAL || qs0 + 31 >= kw0);
  };
  // The four operands of the record, 16 bytes per lane each; a record that is not live is
  // read through an empty resource (zeros, and no branch around the loads).
  // Record of (query head gi, 32-row block qb): rec0 + gi * score_head + qb (records are key-block
  // major, so the row blocks of one key block are consecutive).
  const size_t rec0 =
      (size_t)(b * args.Hq + hkv * group) * args.score_head + score_record(jb, jb, nQ32, CAUSAL) - (size_t)jb;
  auto load_record = [&](const Item& it, bool ok, vec8 (&r)[4]) {
    const int qb = it.qt * 2 + qh;
    const char* base = static_cast<const char*>(args.scores) +
                       (ok ? (rec0 + (size_t)it.gi * args.score_head + (size_t)qb) * kScoreRecordBytes : 0);
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(reinterpret_cast<const u32x4*>(base), ok ? kScoreRecordBytes / 16 : 0);
#pragma unroll
    for (int m = 0; m < 4; ++m)  // read once: non-temporal, as pass 1 wrote them
      r[m] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rs, (m * 64 + lane) * 16, 0, kCachePolicyNt));
  };

  f32x16 dk[C::DT], dv[C::DT];
#pragma unroll
  for (int i = 0; i < C::DT; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }
  vec8 ra[4], rb[4];
  // The walk (without the list): heads in order, each head's tiles from qt_hi down to qt0.
  int gn = work.next_head(0), qn = gn < group ? work.qt_hi(gn) : 0;
  auto advance = [&]() {
    const bool wrap = qn == qt0;
    const int g2 = wrap ? work.next_head(gn + 1) : gn;
    qn = wrap ? (g2 < group ? work.qt_hi(g2) : 0) : qn - 1;
    gn = g2;
  };
  auto item_at = [&](int i) {  // item i; without the list, called for i = 0, 1, 2, ... in turn
    if constexpr (LISTED) {
      return listed(i);
    } else {
      const Item it = walked(gn, qn);
      if (i + 1 < nwork) advance();
      return it;
    }
  };
  bool use = false;  // the current item is live for this wavefront
  if (nwork > 0) {
    const Item it = item_at(0);
    use = live(it);
    issue_tile(it.gi, it.qt, 0);
    load_record(it, use, ra);
  }
  // Tile w: its Q / dO in buffer w & 1, its record in `cur`; the next item is fetched into the
  // other buffer and `nxt`.
  auto step = [&](int w, vec8 (&cur)[4], vec8 (&nxt)[4]) {
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's DMA and record loads of tile w
    __syncthreads();                // every wavefront's DMA of tile w; tile w - 1 no longer read
    bool use_next = false;
    if (w + 1 < nwork) {
      const Item it = item_at(w + 1);
      use_next = live(it);
      issue_tile(it.gi, it.qt, (w + 1) & 1);
      load_record(it, use_next, nxt);
    }
    if (use) {
      const T* __restrict__ tQ = sQ[w & 1];
      const T* __restrict__ tdO = sdO[w & 1];
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const vec8 doa = ld_kmajor<T, false>(tdO, C::LDR, qh * 32 + mh * 16, 8, dt * 32, lane);
          const vec8 qa = ld_kmajor<T, false>(tQ, C::LDR, qh * 32 + mh * 16, 8, dt * 32, lane);
          dv[dt] = M::k16(doa, cur[mh], dv[dt]);
          dk[dt] = M::k16(qa, cur[2 + mh], dk[dt]);
        }
      }
    }
    use = use_next;
  };
  for (int w = 0; w < nwork; w += 2) {
    step(w, ra, rb);
    if (w + 1 < nwork) step(w + 1, rb, ra);
  }

  // The two query halves of a key group: wavefront (kg, 0) finishes dK, (kg, 1) dV.  Each
  // hands the other its partial sum of the other output through LDS.
  __syncthreads();  // every tile read (no DMA is in flight: the last step issued none)
  float* give = reinterpret_cast<float*>(qh ? &sdO[0][0] : &sQ[0][0]) + kg * C::DT * 16 * 64;
  const float* take = reinterpret_cast<const float*>(qh ? &sQ[0][0] : &sdO[0][0]) + kg * C::DT * 16 * 64;
#pragma unroll
  for (int i = 0; i < C::DT; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) give[(i * 16 + r) * 64 + lane] = qh ? dk[i][r] : dv[i][r];
  __syncthreads();
  const int key = kw0 + col;
  if (key < Skv) {
    using vec4 = typename VecOf<T, 4>::type;
    T* __restrict__ out = static_cast<T*>(qh ? args.dv : args.dk) + kvoff + (size_t)key * D;
    const float sc = qh ? 1.0f : args.sm_scale;
#pragma unroll
    for (int i = 0; i < C::DT; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = g * 4 + e;
          v4[e] = ((qh ? dv[i][r] : dk[i][r]) + take[(i * 16 + r) * 64 + lane]) * sc;
        }
        *reinterpret_cast<vec4*>(out + i * 32 + g * 8 + hh * 4) = __builtin_convertvector(v4, vec4);
      }
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwd(const BwdArgs& a, int stages, hipStream_t stream) {
  // The score-store path (BwdArgs::scores set by the caller for the types and head dims
  // that have it) replaces zb / cb with the records and pass 2 with the store kernel.
  constexpr bool kStore = sizeof(T) == 2 && (D == 64 || D == 128);
  const bool store = kStore && a.scores != nullptr;
  static_assert(kStoreBK == kOrderKeyBlock && kPairBK == kOrderKeyBlock, "key_order numbers 64-key blocks");
  if (stages & 1) {
    const int nQB = (a.Sq + kBM - 1) / kBM;
    if (store) {
      if constexpr (kStore)
        hipLaunchKernelGGL((coalibi_bwd_dq_kernel<T, D, CAUSAL, true>), dim3(nQB * a.B * a.Hq), dim3(256), 0, stream,
                           a);
    } else {
      hipLaunchKernelGGL((coalibi_bwd_dq_kernel<T, D, CAUSAL, false>), dim3(nQB * a.B * a.Hq), dim3(256), 0, stream,
                         a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & 2) {
    if (store) {
      if constexpr (kStore) {
        const int nKB = (a.Skv + kStoreBK - 1) / kStoreBK;
        const int nQT = (a.Sq + kStoreBQ - 1) / kStoreBQ;
        if (static_cast<long long>(a.Hq / a.Hkv) * nQT <= kStoreProcessedWords)
          hipLaunchKernelGGL((coalibi_bwd_dkdv_store_kernel<T, D, CAUSAL, true>), dim3(nKB * a.B * a.Hkv), dim3(256),
                             0, stream, a);
        else
          hipLaunchKernelGGL((coalibi_bwd_dkdv_store_kernel<T, D, CAUSAL, false>), dim3(nKB * a.B * a.Hkv),
                             dim3(256), 0, stream, a);
      }
    } else if constexpr (sizeof(T) == 2 && D >= 64) {  // the pair kernel splits D into 32-row halves
      const int nKB = (a.Skv + kPairBK - 1) / kPairBK;
      hipLaunchKernelGGL((coalibi_bwd_dkdv_kernel<T, D, CAUSAL>), dim3(nKB * a.B * a.Hkv), dim3(64 * kPairWaves),
                         0, stream, a);
    } else {
      const int nKB = (a.Skv + kBK - 1) / kBK;
      hipLaunchKernelGGL((coalibi_bwd_dkdv_f32_kernel<T, D, CAUSAL>), dim3(nKB * a.B * a.Hkv), dim3(256), 0,
                         stream, a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

#define COALIBI_INST_BWD(T, D)                                                \
  template hipError_t launch_bwd<T, D, true>(const BwdArgs&, int, hipStream_t); \
  template hipError_t launch_bwd<T, D, false>(const BwdArgs&, int, hipStream_t);

COALIBI_INST_BWD(_Float16, 16)
COALIBI_INST_BWD(_Float16, 32)
COALIBI_INST_BWD(_Float16, 64)
COALIBI_INST_BWD(_Float16, 128)
COALIBI_INST_BWD(_Float16, 256)
COALIBI_INST_BWD(__bf16, 16)
COALIBI_INST_BWD(__bf16, 32)
COALIBI_INST_BWD(__bf16, 64)
COALIBI_INST_BWD(__bf16, 128)
COALIBI_INST_BWD(__bf16, 256)
COALIBI_INST_BWD(float, 16)
COALIBI_INST_BWD(float, 32)
COALIBI_INST_BWD(float, 64)
COALIBI_INST_BWD(float, 128)
COALIBI_INST_BWD(float, 256)

}  // namespace coalibi
