// Launch interface between the C ABI layer and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace coalibi {

constexpr float kLog2eHost = 1.4426950408889634f;

// Tensors are contiguous row-major: q/o/dout/dq (B, Hq, Sq, D),
// k/v/dk/dv (B, Hkv, Skv, D).  Query head h reads key/value head h / (Hq/Hkv).
// zb (penalty statistics written by the forward, read by the backward) is
// (B*Hq, nZB, Sq) fp32 with nZB = ceil(Skv/32): zb[bh][J][i] = sum of
// sigmoid(p_ik) over valid keys k >= 32*J of row i.
struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* slopes;  // (Hq,) penalty slope per query head
  void* o;
  float* lse;  // (B*Hq, Sq) natural-log log-sum-exp
  float* zb;
  int B, Hq, Hkv, Sq, Skv, nZB;
  float sc2;  // sm_scale * log2(e)
};

// Backward scratch: dsum (B*Hq, Sq) holds dO_i . O_i, cb (B*Hq, nZB, Sq)
// holds sum over keys k < 32*J of dA_ik for every 32-key block J.
struct BwdArgs {
  const void* dout;
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const float* lse;
  const float* zb;
  const float* slopes;
  void* dq;
  void* dk;
  void* dv;
  float* dsum;
  float* cb;
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

template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream);

template <typename T, int D>
hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream);

// stages: bit 0 = pass 1 (dq, dsum, cb), bit 1 = pass 2 (dk, dv; needs pass 1's dsum / cb).
template <typename T, int D, bool CAUSAL>
hipError_t launch_bwd(const BwdArgs& a, int stages, hipStream_t stream);

}  // namespace coalibi
