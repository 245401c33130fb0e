// Launch interface between the C ABI layer and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace coalibi {

constexpr float kLog2eHost = 1.4426950408889634f;

// Tensors are contiguous row-major: q/o/dout/dq (B, Hq, Sq, D),
// k/v/dk/dv (B, Hkv, Skv, D).  Query head h reads key/value head h / (Hq/Hkv).
//
// Statistics the forward saves for the backward besides LSE ("stats", int32 / fp32 words,
// O(B*Hq*S) in all):
//   header (kStatsHeader words): word 0 holds flags -- bit 0: row_order is a work order the
//     key-norm launch wrote, bit 1: key_order likewise (without a bit the kernels that would
//     read the table use their fixed order instead), bit 2: the forward ran with the tail
//     skip; the other header words are zero;
//   kstart (B*Hq, nQB) int32, nQB = ceil(Sq/128): the first key the forward processed for
//     each 128-row block (0 when the tail skip is off).  Every key left of it has a softmax
//     weight below 2^-skip_log2 of its row's total in every row of the block (the tail skip
//     below); the backward passes skip the same keys;
//   knorm (B*Hq, nKC) fp32, nKC = ceil(Skv/kNormKeys): max_k |k|_2 over each chunk of
//     kNormKeys keys of key head b*Hkv + h in its first B*Hkv rows, zero in the rest;
//   row_order (B*Hq*nQB) int32: the work order of the forward and pass 1 (below);
//   key_order (B*Hq*nKB) int32, nKB = ceil(Skv/64): the work order of pass 2 over its
//     B*Hkv*nKB key blocks (written, and read, only when Hq == Hkv);
//   rsum (2, B*Hq, Sq) fp32: R_i, the sum of sigmoid(p_ik) over the keys the forward processed
//     (k >= kstart), summed with compensation and saved as hi + lo.  It takes the place of the
//     reference's RowSigTotal (co_alibi_attn.py:37): backward pass 1 walks the keys left to
//     right and rebuilds z at each block start as R minus the sigma it has passed.
//
// Tail skip.  In the log2 domain a row's logit for key k is a_k = t_k - lam2 * z_k with
// t_k = q.k * sm_scale * log2(e) and z_k = sum of sigmoids of the visible keys >= k.  The
// forward walks keys from the diagonal leftwards, so when it has processed every key from
// k_next on, z_k >= zr (the sum over those keys) for every k < k_next, as sigmoids are
// >= 0, and |t_k| <= |q| * max|k| * sm_scale * log2(e) =: bound (Cauchy-Schwarz).  With
// lam2 > 0 and m2 the running maximum, every later weight 2^(a_k - m2) is then at most
// 2^(bound - lam2 * zr - m2); once that is below 2^-skip_log2 for all rows of a 128-row
// block the forward stops.  The row total l is >= 1 at the final scale, so each skipped
// weight is below 2^-skip_log2 of it (the softmax probability s = 2^(a - LSE2) too).
// The threshold follows the type P is rounded to before it multiplies V:
//   fp16: 26 -- P < 2^-26 rounds to zero (below half the smallest subnormal, 2^-25), so
//     the forward's O is bit-identical to the unskipped one;
//   bf16: 32 -- P keeps 8 bits, so each P carries a relative error up to 2^-9; the skipped
//     weights together are below S * 2^-32 of the row total (1e-6 at S = 4096);
//   fp32: 64 -- the validation mode stays within S * 2^-64 of the unskipped result.
// The backward leaves out the same keys; their dA = s (dS - D) terms are below the same
// fraction of the row's scale.
// The skip is a library setting (co_alibi_set_tail_skip, on by default): with it off the
// forward launches no key-norm kernel, processes every key and records kstart = 0.
constexpr int kStatsHeader = 4;
constexpr int kFlagRowOrder = 1;
constexpr int kFlagKeyOrder = 2;
constexpr int kFlagTailSkip = 4;  // the forward ran with the tail skip
constexpr int kNormKeys = 256;
template <typename T>
constexpr float skip_log2() {
  return sizeof(T) == 4 ? 64.0f : (__is_same(T, __bf16) ? 32.0f : 26.0f);
}
constexpr int kSkipRows = 128;  // rows per kstart entry: the forward's and pass 1's row block
// kstart as the backward kernels read it.  It is device data the host cannot check without a
// synchronisation: a value outside [0, Skv] (not written by the forward) counts as 0, so no
// value moves a tile or a record address past the key range.
__device__ __forceinline__ int valid_kstart(int ks, int Skv) { return ks >= 0 && ks <= Skv ? ks : 0; }
inline int stats_kstart_count(int Sq) { return (Sq + kSkipRows - 1) / kSkipRows; }
inline int stats_knorm_count(int Skv) { return (Skv + kNormKeys - 1) / kNormKeys; }
constexpr int kOrderKeyBlock = 64;  // keys per pass-2 work-group (16-bit kernels)
__host__ __device__ inline int stats_key_block_count(int Skv) { return (Skv + kOrderKeyBlock - 1) / kOrderKeyBlock; }

// Work orders.  The tail skip makes a work-group's cost depend on its head's slope: a
// 128-row block of a steep head processes a few key tiles, one of a flat head up to all of
// them.  The hardware hands consecutive work-group ids to the 8 XCDs in turn and, within an
// XCD, to its 4 shader engines in turn, and it dispatches in id order: when the engine
// that the next id is bound for has no free slot, dispatch waits even if other engines are
// idle.  Ids whose costs differ widely (the fixed orders of the kernels) therefore leave
// engines idle; ids in decreasing order of cost keep every engine's queue alike.  The
// key-norm launch writes such orders (coalibi_fwd.hip, schedule_rows / schedule_keys): entry
// j of a table is the item the work-group with id j processes, item = rank * heads + head in
// the fixed order's numbering, sorted by a cost predicted from the slope alone (the order is
// not needed to be exact, only close): a row keeps about W = kOrderWindow / slope keys left
// of its diagonal, where kOrderWindow = (T + 8) / (0.5 log2 e) for the threshold T of the
// type (the sigmoid sum z grows by about 0.5 a key, and the skip fires once slope*z*log2 e
// passes T plus the logit bound, a few units).
// A table is sorted for at most this many items (the sort runs on one wavefront); larger
// grids keep the fixed orders.
constexpr long long kOrderMaxItems = 1 << 20;
inline bool row_order_fits(int B, int Hq, int Sq) {
  return static_cast<long long>(B) * Hq * stats_kstart_count(Sq) <= kOrderMaxItems;
}
inline bool key_order_fits(int B, int Hkv, int Skv) {
  return static_cast<long long>(B) * Hkv * stats_key_block_count(Skv) <= kOrderMaxItems;
}
// Pass 2 follows key_order with one query head per key head only: with grouped heads the
// sorted order measured slower than balanced_item (coalibi_common.h), which keeps runs of key
// blocks of a head on one XCD.
inline bool key_order_used(int B, int Hq, int Hkv, int Skv) { return Hq == Hkv && key_order_fits(B, Hkv, Skv); }
template <typename T>
constexpr float order_window() {
  return (skip_log2<T>() + 8.0f) / (0.5f * kLog2eHost);
}
struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* slopes;  // (Hq,) penalty slope per query head
  void* o;
  float* lse;          // (B*Hq, Sq) natural-log log-sum-exp, or NULL
  int* kstart;         // (B*Hq, nQB), written when not NULL (the backward's statistics)
  const float* knorm;  // (B*Hq, nKC) chunk maxima of |k|, filled before the forward; NULL: no tail skip
  int* flags;          // the statistics' header, written by work-group 0 when not NULL
  int order_flags;     // its flags word: which work orders the key-norm launch wrote
  float* rsum;         // (2, B*Hq, Sq) row sigmoid totals (hi, lo), written when not NULL
  int B, Hq, Hkv, Sq, Skv, nKC;
  float sc2;  // sm_scale * log2(e)
  // Work orders (above): written by the key-norm launch when not NULL (key_order only with
  // row_order); the forward follows row_order when it is sorted (row_order_fits).
  int* row_order;
  int* key_order;
};

// Score store (16-bit types, D = 64 or 128): pass 1 writes the probabilities s and score
// gradients dS of every tile it processes, and pass 2 reduces them into dK and dV instead of
// recomputing them.  One record per (b*Hq + h, 32-key block jb, 32-row block qb) of a pair
// that can be visible: 4096 bytes, the four 16 x 32 B operands of pass 2's products in MFMA
// lane order -- s for rows 0-15, s for rows 16-31, dS for rows 0-15, dS for rows 16-31 of the
// block; in each, lane l holds the 8 rows 8*(l/32) .. +7 of key l%32.  Records are key-block
// major; causal: qb from jb to nQ32 - 1 (a row block below its key block holds no visible
// pair), otherwise every qb.  Records of skipped tiles (tail skip) are never written or read.
constexpr int kScoreRecordBytes = 4096;
// Pass 2 keeps, per query head of a key head's group, one bit per 128-row block (rounded up to
// 64 per head) of whether the forward processed its key block: at most this many 32-bit words.
constexpr int kStoreProcessedWords = 512;
inline bool score_store_fits(int Hq, int Hkv, int Sq) {
  const int wph = (Sq + kSkipRows * 64 - 1) / (kSkipRows * 64) * 2;
  return static_cast<long long>(Hq / Hkv) * wph <= kStoreProcessedWords;
}
__host__ __device__ inline size_t score_record(int jb, int qb, int nQ32, bool causal) {
  if (!causal) return static_cast<size_t>(jb) * nQ32 + qb;
  return static_cast<size_t>(jb) * nQ32 - static_cast<size_t>(jb) * (jb - 1) / 2 + (qb - jb);
}
inline size_t score_records_per_head(int Sq, int Skv, bool causal) {
  const int nQ32 = (Sq + 31) / 32, nJB = (Skv + 31) / 32;
  if (!causal) return static_cast<size_t>(nJB) * nQ32;
  const int J = nJB < nQ32 ? nJB : nQ32;
  return score_record(J, J, nQ32, true);  // records of the blocks before J
}

// Backward scratch: dsum (B*Hq, Sq) holds dO_i . O_i.  The recompute path (pass 2 recomputes s
// and dS) adds zb and cb, (B*Hq, nZB, Sq) fp32 each with nZB = ceil(Skv/32): for every 32-key
// block J, zb[J][i] = sum of sigmoid(p_ik) over the keys k >= 32J of row i and cb[J][i] = sum of
// dA_ik over the keys k < 32J, written by pass 1 for the blocks it processes.  The score-store
// path needs neither.
struct BwdArgs {
  const void* dout;
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const float* lse;
  const float* rsum;  // (2, B*Hq, Sq): the forward's row sigmoid totals, hi and lo parts
  const float* slopes;
  void* dq;
  void* dk;
  void* dv;
  float* dsum;
  float* zb;
  float* cb;
  const int* kstart;  // (B*Hq, nQB): keys left of kstart are skipped (see above)
  const int* flags;   // the forward's flags word: which of the work orders below it wrote
  void* scores;       // score store (above), or NULL: pass 2 recomputes s and dS from zb / cb
  size_t score_head;  // records per (b, h)
  const int* row_order;  // pass 1's work order (above) when flagged, or NULL: the fixed order
  const int* key_order;  // pass 2's work order for 64-key work-groups when flagged, or NULL
  int B, Hq, Hkv, Sq, Skv, nZB;
  float sc2;
  float sm_scale;
};

// Decode: q/o (B, Hq, D); the caches k/v are (B, Hkv, cap, D) with the first L rows
// of every head valid (or the first seq_lens[b] rows of sequence b, at most L).  The
// keys form nChunks chunks of kDecodeChunkKeys; split s of a head covers chunks
// [s*cps, (s+1)*cps).  Split-K partials per (b*Hq + h, split): pmax / psum / psig
// (B*Hq, nSplits) and pout (B*Hq, nSplits, D), fp32.
constexpr int kDecodeChunkKeys = 128;
constexpr int kMaxDecodeGroup = 32;     // query heads per kv head (MFMA tile columns)
constexpr int kMaxDecodeChunks = 16384;  // bounds seq_kv (2^21 keys)
constexpr int kMaxDecodeSplits = 1024;   // split partials per (batch, query head); merge weights in LDS

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* slopes;  // (Hq,)
  void* o;
  float* lse;  // (B*Hq,) or NULL
  float* pmax;
  float* psum;
  float* psig;
  float* pout;
  const int* seq_lens;  // (B,) per-sequence cache lengths, or NULL (all L)
  int B, Hq, Hkv, G, L, cap, nChunks, cps, nSplits;
  float sc2;
};

// Split-K work-groups the decode aims at per CU: one round of the two that are resident.
constexpr int kDecodeWGsPerCU = 2;

// Forward; with a.knorm (the tail skip) it first launches the key-norm kernel that fills it.
template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream);

template <typename T, int D>
hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream);

// stages: bit 0 = pass 1 (dq, dsum, and zb / cb or the score store), bit 1 = pass 2 (dk, dv; needs pass
// 1's output).
template <typename T, int D, bool CAUSAL>
hipError_t launch_bwd(const BwdArgs& a, int stages, hipStream_t stream);

}  // namespace coalibi
