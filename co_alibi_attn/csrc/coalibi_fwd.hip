// Co-ALiBi forward on gfx950.
//
// Semantics follow the reference forward (co_alibi_attn/co_alibi_fwd_kernel.py:46-127
// and model.py:13-40 with the per-head slope of co_alibi_attn.py:147):
//   p_ij   = sm_scale * q_i . k_j
//   s_ij   = sigmoid(p_ij) for valid (i, j), else 0     valid: j < Skv and (!causal or j <= i)
//   z_ij   = sum_{k >= j} s_ik                          (inclusive suffix over keys)
//   a_ij   = p_ij - slope_h * z_ij
//   O_i    = sum_j exp(a_ij - m_i) v_j / (sum_j exp(a_ij - m_i) + 1e-9)
//   LSE_i  = m_i + log(sum_j exp(a_ij - m_i) + 1e-9)
//
// One work-group = 128 query rows of one (batch, query head), 4 wavefronts of
// 32 rows.  Key tiles of 64 are walked from the causal diagonal leftwards so
// the suffix sum z is a running carry.  Per tile and wavefront:
//   S^T = K Q^T   (MFMA, keys on the accumulator rows: with the kRowOfReg
//                  permutation each lane holds 16 consecutive keys of one row)
//   sigmoid, suffix scan (in registers + one exchange with the other half),
//   penalty, online softmax (exp2, lazily rescaled), then
//   O^T += V^T P^T (MFMA, the P accumulators are reused as the B operand).
// K is staged in LDS row-major (rows permuted); V row-major, read as the
// transposed operand with ds_read_b64_tr_b16 (fp32 mode: V stored transposed).
// Besides O and LSE the kernel saves, per 128-row block, the first key it processed
// (kstart, the tail skip's record), and per row the sum R of the sigmoids of the keys it
// processed: backward pass 1 rebuilds z from it.  R is summed in fp64 over 32-key block
// totals, exactly the totals pass 1 computes (the same sigmoids summed in the same order), so
// the difference pass 1 takes is exact up to one rounding.
#include "coalibi_common.h"
#include "coalibi_kernels.h"

namespace coalibi {

namespace {

constexpr int kFwdBM = 128;  // query rows per work-group
constexpr int kFwdBN = 64;   // keys per tile
// Rescale O only when the running max grows by more than 2^8: P stays <= 256,
// exact in fp16/bf16 range, and O/LSE are renormalised to the true max at the end.
constexpr float kRescaleThreshold = 8.0f;

template <typename T, int D>
struct FwdCfg {
  static constexpr bool kTr = sizeof(T) == 2;  // V through LDS transpose reads
  static constexpr int CH = 16 / sizeof(T);
  // O^T is produced in 32-row tiles of the head dim: D = 16 runs on a 32-wide head dim whose
  // upper 16 columns of V are zero in LDS (written once, never loaded over).
  static constexpr int DP = D < 32 ? 32 : D;
  static constexpr int LDK = D + CH;       // sK row stride (elements)
  // sV: row-major [key][d] (stride keeps each 4-row transpose read on distinct
  // banks) or, in fp32 mode, transposed [d][key].
  static constexpr int LDV = kTr ? DP + 2 * CH : kFwdBN + CH;
  static constexpr int V_ELEMS = kTr ? kFwdBN * LDV : DP * LDV;
  static constexpr int KS = D / 16;        // k16 steps over the head dim
  static constexpr int DT = DP / 32;       // 32-row tiles of O^T
};

template <bool MASKED, bool CAUSAL>
__device__ __forceinline__ bool key_ok(int key, int row, int Skv) {
  if (!MASKED) return true;
  return key < Skv && (!CAUSAL || key <= row);
}

// One 64-key tile for one wavefront.  State: acc (O^T, scaled by 2^-m2), m2
// (log2-domain scale, -inf before the first visible key), lsum (this half's
// share of sum_j 2^(a_j - m2)), zr (sigmoid sum of all keys right of the tile, read only).
// Returns the sigmoid totals of the tile's two 32-key blocks, keys k0 + 32.. in btot[1] and k0..
// in btot[0] (the same values in both halves of the wavefront).
template <typename T, int D, bool CAUSAL, bool MASKED>
__device__ __forceinline__ void fwd_tile(const T* __restrict__ sK, const T* __restrict__ sV,
                                         const typename Mfma<T>::vec8 (&qf)[FwdCfg<T, D>::KS],
                                         f32x16 (&acc)[FwdCfg<T, D>::DT], float& m2, float& lsum,
                                         float zr, float (&btot)[2], int k0, int row, int lane, int Skv,
                                         float sc2, float lam2) {
  using C = FwdCfg<T, D>;
  using M = Mfma<T>;
  const int col = lane & 31, hh = lane >> 5;

  // S^T tile: two 32-key subtiles; register r of subtile st <-> key k0 + st*32 + hh*16 + r.
  f32x16 sacc[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    sacc[st] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
      sacc[st] = M::k16(ld_vec8(sK + (st * 32 + col) * C::LDK + ks * 16 + hh * 8), qf[ks], sacc[st]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // sigma and its inclusive suffix sum inside each lane's 16-key run.
  float loc[2][16];
  float tot[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    float run = 0.f;
#pragma unroll
    for (int r = 15; r >= 0; --r) {
      float s = sigmoid_log2(sacc[st][r] * sc2);
      if (MASKED) s = key_ok<MASKED, CAUSAL>(k0 + st * 32 + hh * 16 + r, row, Skv) ? s : 0.f;
      run += s;
      loc[st][r] = run;
    }
    tot[st] = run;
  }
  // Run totals in key order (right to left): (1,1) (1,0) (0,1) (0,0), where (st, h) is
  // the 16-key run of subtile st held by wavefront half h.
  const float oth0 = other_half(tot[0]), oth1 = other_half(tot[1]);
  const float T11 = hh ? tot[1] : oth1, T10 = hh ? oth1 : tot[1];
  const float T01 = hh ? tot[0] : oth0, T00 = hh ? oth0 : tot[0];
  const float zst1 = (zr + T11) + T10;  // suffix sum from key k0 + 32
  const float off[2] = {hh ? zst1 : zst1 + T01, hh ? zr : zr + T11};
  btot[1] = T11 + T10;
  btot[0] = T01 + T00;

  // Log2-domain logit relative to the current scale:
  //   t - lam2 * (off + loc) - mb = fma(-lam2, loc, fma(s, sc2, -(mb + lam2 * off)))
  const float mb = m2 == kNegInf ? 0.f : m2;
  float mt = kNegInf;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const float cst = mb + lam2 * off[st];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float av = fmaf(-lam2, loc[st][r], fmaf(sacc[st][r], sc2, -cst));
      if (MASKED) av = key_ok<MASKED, CAUSAL>(k0 + st * 32 + hh * 16 + r, row, Skv) ? av : kNegInf;
      sacc[st][r] = av;
      mt = fmaxf(mt, av);
    }
  }
  mt = fmaxf(mt, other_half(mt));
  const bool need = m2 == kNegInf ? mt > kNegInf : mt > kRescaleThreshold;
  if (__any(need)) {
    const float delta = need ? mt : 0.f;
    const float alpha = need ? (m2 == kNegInf ? 0.f : fast_exp2(-delta)) : 1.f;
    m2 = need ? mb + delta : m2;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
#pragma unroll
    for (int st = 0; st < 2; ++st) sacc[st] -= delta;
  }

  typename M::vec8 pb[2][2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int mh = 0; mh < 2; ++mh) {
      f32x8 pv;
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = fast_exp2(sacc[st][mh * 8 + e]);
      pb[st][mh] = M::pack(pv);
      lsum = sum8(pb[st][mh], lsum);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // O^T[d][q] += V^T[d][key] P^T[key][q]; A rows are keys st*32 + hh*16 + mh*8 + e.
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        typename M::vec8 va;
        if constexpr (C::kTr)
          va = ld_kmajor<T, false>(sV, C::LDV, st * 32 + mh * 8, 16, dt * 32, lane);
        else
          va = ld_vec8(sV + (dt * 32 + col) * C::LDV + st * 32 + hh * 16 + mh * 8);
        acc[dt] = M::k16(va, pb[st][mh], acc[dt]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Work orders (coalibi_kernels.h), written by the first work-groups of the key-norm launch:
// one sorts the forward's and pass 1's row blocks, one pass 2's key blocks, largest
// predicted cost first.
constexpr int kOrderBuckets = 256;  // cost classes: ceil(extent / 256) keys or rows each
constexpr int kOrderLdsHeads = 1024;

struct ScheduleArgs {
  const float* slopes;
  int* row_order;  // NULL: not written
  int* key_order;  // NULL: not written
  int B, Hq, Hkv, Sq, Skv;
  int causal;
  int rows_sorted, keys_sorted;  // 0: the table holds its index order (too large to sort, or unused)
  float window;                  // order_window<T>()
};

// The lanes of the wavefront whose `b` equals this lane's (among the lanes with `ok`), matched
// bit by bit with ballots.
__device__ __forceinline__ unsigned long long same_bucket(int b, bool ok) {
  unsigned long long peers = __ballot(ok);
#pragma unroll
  for (int bit = 0; (1 << bit) < kOrderBuckets; ++bit) {
    const bool one = (b >> bit) & 1;
    const unsigned long long m = __ballot(one);
    peers &= one ? m : ~m;
  }
  return peers;
}

// Stable counting sort by one work-group of 256 threads: out[j] is the j-th of the n items in
// decreasing bucket order, the items of one bucket in index order.  Wavefront w takes the w-th
// quarter of the items; per wavefront, a chunk of 64 items is counted (and later placed) with
// one LDS update per distinct bucket, by the lowest lane that holds it.  lds: 5 *
// kOrderBuckets ints.
template <typename F>
__device__ void sort_items_desc(int n, const F& bucket, int* __restrict__ out, int* lds, int tid) {
  constexpr int K = kOrderBuckets;
  static_assert(K == 256, "one thread per bucket in the scan");
  int* const cur = lds;          // [4][K]: per-wavefront counts, then per-wavefront cursors
  int* const part = lds + 4 * K;  // [4]: per-wavefront scan totals
  const int lane = tid & 63, wave = tid >> 6;
  for (int j = tid; j < 4 * K; j += 256) cur[j] = 0;
  __syncthreads();
  const int per = (n + 3) / 4;
  const int lo = min(wave * per, n), hi = min(lo + per, n);
  int* const mine = cur + wave * K;
  for (int base = lo; base < hi; base += 64) {
    const int i = base + lane;
    const bool ok = i < hi;
    const int b = ok ? bucket(i) : 0;
    const unsigned long long peers = same_bucket(b, ok);
    if (ok && __popcll(peers & ((1ull << lane) - 1)) == 0) mine[b] += __popcll(peers);
  }
  __syncthreads();
  // Thread t owns bucket K - 1 - t (descending): its total over the wavefronts, an exclusive
  // scan over the threads, then each wavefront's cursor for the bucket.
  const int bk = K - 1 - tid;
  int c[4], tot = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) tot += (c[w] = cur[w * K + bk]);
  int incl = tot;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) part[wave] = incl;
  __syncthreads();
  int start = incl - tot;
  for (int w = 0; w < wave; ++w) start += part[w];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    cur[w * K + bk] = start;
    start += c[w];
  }
  __syncthreads();
  for (int base = lo; base < hi; base += 64) {
    const int i = base + lane;
    const bool ok = i < hi;
    const int b = ok ? bucket(i) : 0;
    const unsigned long long peers = same_bucket(b, ok);
    if (ok) {
      // LDS operations of the wavefront complete in program order: every lane reads the
      // cursor before its lowest lane moves it.
      const int before = __popcll(peers & ((1ull << lane) - 1));
      const int at = mine[b];
      out[at + before] = i;
      if (before == 0) mine[b] = at + __popcll(peers);
    }
  }
}

// Per query head, the keys (or rows) a row block (or key block) keeps at most: window / slope,
// or +inf for a slope that skips nothing (<= 0 or NaN).  Held in LDS for the first
// kOrderLdsHeads heads; the others are computed where they are needed.
struct HeadWindow {
  const float* __restrict__ slopes;
  const float* lds;
  float window;
  __device__ float operator()(int h) const {
    if (h < kOrderLdsHeads) return lds[h];
    const float lam = slopes[h];
    return lam > 0.f ? window / lam : __builtin_inff();
  }
};

// Cost class of a row block (item rank * heads + bh, rank 0 = the last row block): the keys
// it processes, up to its diagonal (causal) and at most its head's window, in units of
// ceil(Skv / kOrderBuckets) keys.
struct RowCost {
  HeadWindow win;
  int heads, Hq, nQB, Skv, causal;
  float unit;
  __device__ int operator()(int i) const {
    const int rank = i / heads, bh = i - rank * heads;
    const int qb = nQB - 1 - rank;
    const float keys = causal ? (float)min((qb + 1) * kSkipRows, Skv) : (float)Skv;
    return min((int)(fminf(keys, win(bh % Hq)) / unit), kOrderBuckets - 1);
  }
};

// Cost class of a 64-key block (item kb * heads + bh; one query head per key head): the query
// rows that see it (causal: rows from its first key on), at most the head's window, in units
// of ceil(Sq / kOrderBuckets) rows.
struct KeyCost {
  HeadWindow win;
  int heads, H, Sq, causal;
  float unit;
  __device__ int operator()(int i) const {
    const int kb = i / heads, bh = i - kb * heads;
    const float rows = causal ? (float)max(Sq - kb * kOrderKeyBlock, 0) : (float)Sq;
    return min((int)(fminf(rows, win(bh % H)) / unit), kOrderBuckets - 1);
  }
};

// Work-group 0 writes the row order, work-group 1 the key order.  Every element of both tables
// is written (the statistics are an output): a table that is not sorted holds its index order,
// and the key table's room for B*Hq*nKB entries past its B*Hkv*nKB items holds zeros.
__device__ void schedule_orders(const ScheduleArgs& s, int which, int tid) {
  __shared__ int lds[5 * kOrderBuckets];
  __shared__ float wlds[kOrderLdsHeads];
  for (int h = tid; h < min(s.Hq, kOrderLdsHeads); h += 256) {
    const float lam = s.slopes[h];
    wlds[h] = lam > 0.f ? s.window / lam : __builtin_inff();
  }
  __syncthreads();
  const HeadWindow win{s.slopes, wlds, s.window};
  if (which == 0) {
    const int nQB = (s.Sq + kSkipRows - 1) / kSkipRows;
    const int n = nQB * s.B * s.Hq;
    if (s.rows_sorted) {
      const RowCost cost{win, s.B * s.Hq, s.Hq, nQB, s.Skv, s.causal,
                         (float)((s.Skv + kOrderBuckets - 1) / kOrderBuckets)};
      sort_items_desc(n, cost, s.row_order, lds, tid);
    } else {
      for (int i = tid; i < n; i += 256) s.row_order[i] = i;
    }
  } else {
    const int nKB = stats_key_block_count(s.Skv);
    const int n = nKB * s.B * s.Hkv;
    if (s.keys_sorted) {
      const KeyCost cost{win, s.B * s.Hkv, s.Hkv, s.Sq, s.causal,
                         (float)((s.Sq + kOrderBuckets - 1) / kOrderBuckets)};
      sort_items_desc(n, cost, s.key_order, lds, tid);
    } else {
      for (int i = tid; i < n; i += 256) s.key_order[i] = i;
    }
    for (int i = n + tid; i < nKB * s.B * s.Hq; i += 256) s.key_order[i] = 0;
  }
}

// max over each chunk of kNormKeys keys of |k|_2, per key head: the key side of the tail
// skip's bound.  One work-group per (head, chunk) over B*Hq heads: the buffer has room for
// B*Hq rows, and rows past the B*Hkv key heads are written as zero, so every element of
// the forward's statistics is written (deterministic outputs).  The D/CH lanes that hold one key row's 16-byte chunks
// sum their squares with xor shuffles.  A NaN norm is kept (fmaxf would drop it), so a
// non-finite key disables the skip for its head.
// The first nSched work-groups of the launch write the work orders instead.
template <typename T, int D>
__global__ __launch_bounds__(256) void coalibi_key_norm_kernel(const T* __restrict__ k, float* __restrict__ knorm,
                                                               int Skv, int nKC, int nKeyHeads, int nSched,
                                                               ScheduleArgs sched) {
  constexpr int CH = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int CPR = D / CH;              // chunks (lanes) per key row: 2 .. 32
  constexpr int RPP = 256 / CPR;           // key rows per pass of the work-group
  static_assert(CPR >= 2 && CPR <= 64 && (CPR & (CPR - 1)) == 0, "a key row spans a power-of-two lane group");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if ((int)blockIdx.x < nSched) {
    schedule_orders(sched, blockIdx.x, tid);
    return;
  }
  const int id = blockIdx.x - nSched;
  const int bhk = id / nKC, c = id - bhk * nKC;
  if (bhk >= nKeyHeads) {
    if (tid == 0) knorm[(size_t)bhk * nKC + c] = 0.f;
    return;
  }
  // Every load of the chunk goes out before any is used, through a buffer resource over the
  // chunk's valid rows (rows past Skv read as zero, whose norm 0 leaves the maximum alone).
  constexpr int NP = kNormKeys / RPP;  // passes over the chunk
  const int r0 = c * kNormKeys;
  const __amdgpu_buffer_rsrc_t rs = tile_rsrc(k + ((size_t)bhk * Skv + r0) * D, min(kNormKeys, Skv - r0) * D);
  u32x4 x[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p)
    x[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, ((p * RPP + tid / CPR) * D + (tid % CPR) * CH) * (int)sizeof(T),
                                                 0, 0);
  float best = 0.f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const typename VecOf<T, CH>::type xv = __builtin_bit_cast(typename VecOf<T, CH>::type, x[p]);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < CH; ++e) ss = fmaf((float)xv[e], (float)xv[e], ss);
#pragma unroll
    for (int off = CPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    best = ss != ss ? ss : fmaxf(best, ss);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(best, off);
    best = o != o ? o : fmaxf(best, o);
  }
  __shared__ float red[4];
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (tid == 0) {
    float m = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = red[w] != red[w] ? red[w] : fmaxf(m, red[w]);
    knorm[(size_t)bhk * nKC + c] = sqrtf(m);
  }
}

// SKIP: the tail skip (args.knorm holds the key norms); without it every key is processed and
// the kernel carries none of the skip's per-tile test.
template <typename T, int D, bool CAUSAL, bool SKIP>
__global__ __launch_bounds__(256, (sizeof(T) == 4 || D > 128) ? 1 : 2) void coalibi_fwd_kernel(FwdArgs args) {
  using C = FwdCfg<T, D>;
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  using KTile = TileLoader<T, D, kFwdBN>;
  using VTile = TileLoader<T, D, kFwdBN, !FwdCfg<T, D>::kTr>;
  __shared__ __align__(16) T sK[kFwdBN * C::LDK];
  __shared__ __align__(16) T sV[C::V_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int Sq = args.Sq, Skv = args.Skv;
  const int nQB = (Sq + kFwdBM - 1) / kFwdBM;
  const WorkItem item = args.row_order ? table_item(args.row_order, blockIdx.x, args.B * args.Hq, gridDim.x)
                                       : lpt_item(blockIdx.x, args.B * args.Hq, 1);
  const int bh = item.head;
  const int qb = nQB - 1 - item.rank;  // rank 0: the longest causal rows
  const int b = bh / args.Hq, hq = bh - b * args.Hq;
  const int hkv = hq / (args.Hq / args.Hkv);
  const T* __restrict__ Qp = static_cast<const T*>(args.q) + (size_t)bh * Sq * D;
  const size_t kvoff = ((size_t)b * args.Hkv + hkv) * (size_t)Skv * D;
  const T* __restrict__ Kp = static_cast<const T*>(args.k) + kvoff;
  const T* __restrict__ Vp = static_cast<const T*>(args.v) + kvoff;
  const float lam2 = args.slopes[hq] * kLog2e;
  const float sc2 = args.sc2;
  if constexpr (D < C::DP) {  // the padding columns of V stay zero: tiles only write the D real ones
    lds_zero(sV, (int)sizeof(sV), tid, 256);
  }

  const int q0 = qb * kFwdBM;
  const int wrow0 = q0 + wave * 32;
  const int row = wrow0 + col;
  const bool row_ok = row < Sq;

  // 16-bit types: Q pre-scaled by sm_scale*log2(e) (one rounding per element, far below the
  // input precision's effect on q.k), so the tile math takes the scale 1 and multiplies by nothing.
  constexpr bool kPreScaled = sizeof(T) == 2;
  // The reads before the first tile go out together and share one round trip: the Q
  // fragments, the first K / V tile and (tail skip) the key-norm chunk maxima.
  // Q through a buffer resource over the block's valid rows: rows past Sq read as zero.
  vec8 qf[C::KS];
  {
    const __amdgpu_buffer_rsrc_t qrs = tile_rsrc(Qp + (size_t)q0 * D, min(Sq - q0, kFwdBM) * D);
    const int qoffb = ((wave * 32 + col) * D + hh * 8) * (int)sizeof(T);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) qf[ks] = buffer_load_vec8<vec8>(qrs, qoffb + ks * 16 * (int)sizeof(T));
  }
  const int last_key = CAUSAL ? min(q0 + kFwdBM - 1, Skv - 1) : Skv - 1;
  const int nkt = last_key / kFwdBN + 1;
  KTile kt_regs;
  VTile vt_regs;
  kt_regs.load(Kp, (nkt - 1) * kFwdBN, Skv, tid);
  vt_regs.load(Vp, (nkt - 1) * kFwdBN, Skv, tid);
  const bool tail_skip = SKIP && lam2 > 0.f;
  float km = 0.f;
  if (tail_skip) {
    const float* kn = args.knorm + ((size_t)b * args.Hkv + hkv) * args.nKC;
    for (int c = tid; c < args.nKC; c += 256) km = kn[c] != kn[c] ? kn[c] : fmaxf(km, kn[c]);
  }
  if constexpr (kPreScaled) {
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) qf[ks] = scale_vec8<T>(qf[ks], sc2);
  }
  const float tile_sc2 = kPreScaled ? 1.0f : sc2;

  // Tail skip (coalibi_kernels.h): this row's bound on |t| in log2 units, |q| * max|k| with
  // the scale (folded into q in 16-bit types), with a margin for the rounding of the norms
  // and of the fp32 dot products.
  // The bound stays in LDS (one per row) rather than in a register across the tile loop.
  __shared__ float sKmax[4];
  __shared__ float sBound[kFwdBM];
  __shared__ int sDone[4];
  if (tail_skip) {
    float qq = 0.f;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) qq = fmaf((float)qf[ks][e], (float)qf[ks][e], qq);
    qq += other_half(qq);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float o = __shfl_xor(km, off);
      km = o != o ? o : fmaxf(km, o);
    }
    if (lane == 0) sKmax[wave] = km;
    __syncthreads();
    km = sKmax[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) km = sKmax[w] != sKmax[w] ? sKmax[w] : fmaxf(km, sKmax[w]);
    if (hh == 0) sBound[wave * 32 + col] = sqrtf(qq) * km * (kPreScaled ? 1.0f : sc2) * 1.001f + 1e-3f;
  }
  int kfirst = 0;  // first key of the leftmost tile processed

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  // zsum: the sigmoid sum of the keys processed so far (right of the current tile), in fp64;
  // zr, its fp32 value, is the running offset of the tile's z.
  float m2 = kNegInf, lsum = 0.f, zr = 0.f;
  double zsum = 0.0;
  if (args.flags != nullptr && blockIdx.x == 0 && tid < kStatsHeader) args.flags[tid] = tid == 0 ? args.order_flags : 0;

  int kt_end = 0;  // the loop's lower bound, raised by the tail skip
  for (int kt = nkt - 1; kt >= kt_end; --kt) {
    __syncthreads();
    // Every wavefront's rows passed the tail test after tile kt + 1: the keys left of it
    // carry weights below 2^-skip_log2<T>() (the vote is uniform, so all wavefronts leave here).
    // Leaving through the loop bound rather than a break keeps the loop's register
    // allocation as it is without the skip (a break costs 13 spilled registers at D = 128).
    if (tail_skip && kt < nkt - 1 && (sDone[0] & sDone[1] & sDone[2] & sDone[3])) {
      kfirst = (kt + 1) * kFwdBN;
      kt_end = kt + 1;
      continue;
    }
    kt_regs.store_rows(sK, C::LDK, tid);
    if constexpr (C::kTr)
      vt_regs.template store_rows<false>(sV, C::LDV, tid);
    else
      vt_regs.store_cols(sV, C::LDV, tid);
    __syncthreads();
    // The next tile's K / V go into registers during this tile's math; at D = 256 those
    // registers do not fit beside the tile state, and the loads are issued after it.
    constexpr bool kPrefetchKV = D <= 128;
    if (kPrefetchKV && kt > 0) {
      kt_regs.load(Kp, (kt - 1) * kFwdBN, Skv, tid);
      vt_regs.load(Vp, (kt - 1) * kFwdBN, Skv, tid);
    }
    const int k0 = kt * kFwdBN;
    const bool skip = CAUSAL && k0 > wrow0 + 31;  // every key of the tile is above this wavefront's rows
    if (skip) {
      if (!kPrefetchKV && kt > 0) {
        kt_regs.load(Kp, (kt - 1) * kFwdBN, Skv, tid);
        vt_regs.load(Vp, (kt - 1) * kFwdBN, Skv, tid);
      }
      if (tail_skip && lane == 0) sDone[wave] = Sq <= wrow0;  // no visible key yet: only rows past Sq pass
      continue;
    }
    const bool masked = (CAUSAL && k0 + kFwdBN - 1 > wrow0) || (k0 + kFwdBN > Skv);
    float btot[2];
    if (masked)
      fwd_tile<T, D, CAUSAL, true>(sK, sV, qf, acc, m2, lsum, zr, btot, k0, row, lane, Skv, tile_sc2, lam2);
    else
      fwd_tile<T, D, CAUSAL, false>(sK, sV, qf, acc, m2, lsum, zr, btot, k0, row, lane, Skv, tile_sc2, lam2);
    zsum += (double)btot[1];  // right block first, as the keys are walked
    zsum += (double)btot[0];
    zr = (float)zsum;
    if (!kPrefetchKV && kt > 0) {
      kt_regs.load(Kp, (kt - 1) * kFwdBN, Skv, tid);
      vt_regs.load(Vp, (kt - 1) * kFwdBN, Skv, tid);
    }
    if (tail_skip) {
      // Every key left of k0 has z >= zr, so its weight is at most 2^(bound - lam2*zr - m2).
      const bool done =
          !row_ok || (m2 != kNegInf && sBound[wave * 32 + col] - lam2 * zr - m2 < -skip_log2<T>());
      const bool all = __all(done);
      if (lane == 0) sDone[wave] = all;
    }
  }
  if (args.kstart != nullptr && tid == 0) args.kstart[(size_t)bh * nQB + qb] = kfirst;

  // O = acc / l and LSE = m + log(l) with l = sum_j 2^(a_j - m2) >= 1 (m2 is one of
  // the a_j and at most 8 below their max): the reference's "+1e-9" in l + 1e-9
  // (co_alibi_fwd_kernel.py:115,120) is below fp32 resolution and is omitted.
  const float ltot = lsum + other_half(lsum);
  const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
  if (row_ok) {
    T* __restrict__ Orow = static_cast<T*>(args.o) + ((size_t)bh * Sq + row) * D;
    using vec4 = typename VecOf<T, 4>::type;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (dt * 32 + g * 8 >= D) continue;  // padding rows of O^T (D = 16)
        f32x4 v4 = {acc[dt][g * 4 + 0] * inv, acc[dt][g * 4 + 1] * inv, acc[dt][g * 4 + 2] * inv,
                    acc[dt][g * 4 + 3] * inv};
        *reinterpret_cast<vec4*>(Orow + dt * 32 + g * 8 + hh * 4) = __builtin_convertvector(v4, vec4);
      }
    }
    if (hh == 0 && args.lse != nullptr)
      args.lse[(size_t)bh * Sq + row] = ltot > 0.f ? (m2 + log2f(ltot)) * kLn2 : kNegInf;
    if (hh == 0 && args.rsum != nullptr) {  // R as hi + lo, exact to about 2^-48 of it
      const float hi = (float)zsum;
      args.rsum[(size_t)bh * Sq + row] = hi;
      args.rsum[(size_t)args.B * args.Hq * Sq + (size_t)bh * Sq + row] = (float)(zsum - (double)hi);
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  static_assert(kFwdBM == kSkipRows, "kstart entries are per forward row block");
  FwdArgs f = a;
  const bool rows_sorted = row_order_fits(a.B, a.Hq, a.Sq);
  f.order_flags = 0;
  if (a.knorm != nullptr) {
    const bool keys_sorted = key_order_used(a.B, a.Hq, a.Hkv, a.Skv);
    const ScheduleArgs sched{a.slopes, a.row_order, a.key_order, a.B, a.Hq, a.Hkv, a.Sq, a.Skv, CAUSAL ? 1 : 0,
                             rows_sorted ? 1 : 0, keys_sorted ? 1 : 0, order_window<T>()};
    // The key table needs the row table's work-group before it (work-group 1 writes it).
    const int nSched = a.row_order == nullptr ? 0 : (a.key_order != nullptr ? 2 : 1);
    hipLaunchKernelGGL((coalibi_key_norm_kernel<T, D>), dim3(nSched + a.nKC * a.B * a.Hq), dim3(256), 0, stream,
                       static_cast<const T*>(a.k), const_cast<float*>(a.knorm), a.Skv, a.nKC, a.B * a.Hkv, nSched,
                       sched);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // The backward follows a table only where it was sorted; an unsorted one holds the index
    // order, which the fixed orders of the kernels beat (their heads rotate over the XCDs).
    if (a.row_order != nullptr && rows_sorted) f.order_flags |= kFlagRowOrder;
    if (a.key_order != nullptr && keys_sorted) f.order_flags |= kFlagKeyOrder;
    f.order_flags |= kFlagTailSkip;
  }
  if (a.knorm == nullptr || !rows_sorted) f.row_order = nullptr;  // no sorted table: the fixed order
  const int nQB = (a.Sq + kFwdBM - 1) / kFwdBM;
  const int grid = nQB * a.B * a.Hq;
  if (a.knorm != nullptr)
    hipLaunchKernelGGL((coalibi_fwd_kernel<T, D, CAUSAL, true>), dim3(grid), dim3(256), 0, stream, f);
  else
    hipLaunchKernelGGL((coalibi_fwd_kernel<T, D, CAUSAL, false>), dim3(grid), dim3(256), 0, stream, f);
  return hipGetLastError();
}

#define COALIBI_INST_FWD(T, D)                                           \
  template hipError_t launch_fwd<T, D, true>(const FwdArgs&, hipStream_t); \
  template hipError_t launch_fwd<T, D, false>(const FwdArgs&, hipStream_t);

COALIBI_INST_FWD(_Float16, 16)
COALIBI_INST_FWD(_Float16, 32)
COALIBI_INST_FWD(_Float16, 64)
COALIBI_INST_FWD(_Float16, 128)
COALIBI_INST_FWD(_Float16, 256)
COALIBI_INST_FWD(__bf16, 16)
COALIBI_INST_FWD(__bf16, 32)
COALIBI_INST_FWD(__bf16, 64)
COALIBI_INST_FWD(__bf16, 128)
COALIBI_INST_FWD(__bf16, 256)
COALIBI_INST_FWD(float, 16)
COALIBI_INST_FWD(float, 32)
COALIBI_INST_FWD(float, 64)
COALIBI_INST_FWD(float, 128)
COALIBI_INST_FWD(float, 256)

}  // namespace coalibi
