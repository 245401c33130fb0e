// Co-ALiBi decode on gfx950: one new query per (batch, query head) against a key /
// value cache holding L positions, every one of them visible.  In the reference's
// convention (top-left causal alignment, co_alibi_attn/co_alibi_fwd_kernel.py:80-90)
// this is the op with causal=False and Sq = 1:
//   t_j = sm_scale*log2(e) * q.k_j,   sigma_j = sigmoid(t_j / log2(e)),
//   z_j = sum_{k >= j} sigma_k,       a_j = t_j - slope*log2(e) * z_j,
//   O   = sum_j 2^(a_j - m) v_j / sum_j 2^(a_j - m),   LSE = (m + log2 l) * ln 2.
//
// Decode reads the whole cache once for O(L*D) flops per query head: it is bound by
// HBM bandwidth.  The keys are split into chunks of 256 (split-K) so that every CU
// streams a part of the cache, and two kernels run:
//   1. split: per (chunk, batch, kv head), all query heads of the group at once.
//      S^T = K_chunk Q^T on MFMA (keys on the accumulator rows, the group's query
//      heads on the columns), z from the sigma suffix inside the chunk only, the
//      chunk's softmax partial (max, sum, O = P V on MFMA) and its sigma total.
//   2. merge: per (batch, query head).  The keys after chunk c add the same amount
//      off_c = sum_{c' > c} sigma_total[c'] to z_j of every key of chunk c, which
//      shifts a_j of the whole chunk by -slope*log2(e)*off_c and leaves its sum and
//      O partial unchanged once the maximum is shifted by the same amount.  The
//      merge therefore scans the chunk sigma totals, shifts the chunk maxima and
//      combines the partials with the usual rescaling.
// K is read straight into MFMA fragments with buffer loads; V goes to LDS by
// buffer-to-LDS DMA, issued first so that it overlaps the score products, and is read
// back as the k-major B operand of P V.
#include "coalibi_common.h"
#include "coalibi_kernels.h"

namespace coalibi {

namespace {

constexpr int kDecWaves = 4;
constexpr int kDecWaveKeys = 64;                      // keys per wavefront: two 32-key MFMA tiles
constexpr int kDecMergeThreads = 256;
static_assert(kDecWaves * kDecWaveKeys == kDecodeChunkKeys, "chunk = the work-group's keys");

template <typename T, int D>
struct DecCfg {
  // V row stride in LDS (elements): the transpose-read layout of the forward for 16-bit,
  // one 16-byte pad for fp32 (read element-wise).
  static constexpr int LD = sizeof(T) == 2 ? D + 16 : D + 4;
  static constexpr int KS = D / 16;  // k16 steps over the head dim
  static constexpr int DT = D / 32;  // 32-column tiles of O
  static constexpr int WAVE_ELEMS = kDecWaveKeys * LD;
  static_assert(kMaxDecodeGroup * D * 4 <= WAVE_ELEMS * (int)sizeof(T), "O partials alias the V tile");
};

// Eight consecutive elements of a row of T through a buffer resource.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec8 buf_vec8(__amdgpu_buffer_rsrc_t r, int byte_off) {
  if constexpr (sizeof(T) == 2) {
    return __builtin_bit_cast(typename Mfma<T>::vec8, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
  } else {
    typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
    const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off + 16, 0, 0);
    return __builtin_bit_cast(f32x8, u32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
  }
}

// k-major operand: lane l receives tile[rbase + (l/32)*khs + e][col0 + l%32], e = 0..7.
// Transpose reads for 16-bit; fp32 reads the eight elements one by one.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec8 ld_kmajor_dec(const T* tile, int ld, int rbase, int khs,
                                                                  int col0, int lane) {
  if constexpr (sizeof(T) == 2) {
    return ld_kmajor<T, false>(tile, ld, rbase, khs, col0, lane);
  } else {
    const T* p = tile + (rbase + (lane >> 5) * khs) * ld + col0 + (lane & 31);
    typename Mfma<T>::vec8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = p[e * ld];
    return v;
  }
}

// s_waitcnt immediate that waits until at most n vector-memory operations are outstanding
// and leaves the LDS / export counters alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <typename T, int D>
__global__ __launch_bounds__(kDecWaves * 64, D > 128 ? 1 : 2) void coalibi_decode_split_kernel(DecodeArgs a) {
  using M = Mfma<T>;
  using V8 = typename M::vec8;
  using C = DecCfg<T, D>;
  constexpr int kKLoads = 2 * C::KS * (sizeof(T) == 4 ? 2 : 1);  // buffer loads per K fragment set
  // The next chunk's K loads during this chunk's math; at D = 256 its registers do not
  // fit beside the chunk state and it is loaded after P V instead.
  constexpr bool kPrefetch = D <= 128;
  __shared__ __align__(16) T sV[kDecWaves * C::WAVE_ELEMS];
  __shared__ float sSig[2][kDecWaves][kMaxDecodeGroup];  // per-wavefront sigma totals (by chunk parity)
  __shared__ float sMax[kDecWaves][kMaxDecodeGroup];
  __shared__ float sSum[kDecWaves][kMaxDecodeGroup];
  __shared__ float sScale[kDecWaves][kMaxDecodeGroup];
  __shared__ __align__(16) float sFold[kDecWaves][kMaxDecodeGroup];  // per-chunk rescale by head

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane & 31, hh = lane >> 5;
  const int split = blockIdx.x, bhk = blockIdx.y;
  const int G = a.G, nS = a.nSplits;
  const int b = bhk / a.Hkv, hkv = bhk - b * a.Hkv;
  // This sequence's cache length (per-sequence lengths clamped to [0, L]).
  const int L = a.seq_lens == nullptr ? a.L : min(max(a.seq_lens[b], 0), a.L);
  const int hq0 = hkv * G;  // first query head of the group
  const size_t bh0 = (size_t)b * a.Hq + hq0;
  const int c_first = split * a.cps;
  const int c_last = min(c_first + a.cps, (L + kDecodeChunkKeys - 1) / kDecodeChunkKeys) - 1;
  if (c_last < c_first) {  // the split lies past this sequence's length: an empty partial
    for (int i = tid; i < G * D; i += kDecWaves * 64) a.pout[((bh0 + i / D) * nS + split) * D + i % D] = 0.f;
    if (tid < G) {
      const size_t pi = (bh0 + tid) * nS + split;
      a.pmax[pi] = kNegInf;
      a.psum[pi] = 0.f;
      a.psig[pi] = 0.f;
    }
    return;
  }
  const T* const kbase = static_cast<const T*>(a.k) + (size_t)bhk * a.cap * D;
  const T* const vbase = static_cast<const T*>(a.v) + (size_t)bhk * a.cap * D;
  T* const sVw = sV + wave * C::WAVE_ELEMS;
  const bool head_ok = hl < G;
  const int hsafe = head_ok ? hl : 0;
  const float lam2 = a.slopes[hq0 + hsafe] * kLog2e;

  // K fragments of chunk c: A row R of tile i holds key 32*i + kRowOfReg(R), so register r
  // of lane l ends up with key 32*i + 16*(l/32) + r of the wavefront.  Keys past L read 0.
  auto load_k_tile = [&](V8 (&dst)[C::KS], int c, int i) {
    const int row0 = c * kDecodeChunkKeys + wave * kDecWaveKeys;
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kbase + (size_t)row0 * D, min(max(L - row0, 0), kDecWaveKeys) * D);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks)
      dst[ks] = buf_vec8<T>(kr, ((32 * i + kRowOfReg(hl)) * D + ks * 16 + hh * 8) * (int)sizeof(T));
  };
  // V rows row0.. of this wavefront -> its LDS tile by buffer-to-LDS DMA; each instruction
  // writes 64 consecutive 16-byte chunks of the padded tile.  Pad chunks and rows past L
  // point past the resource and land as zeros.  Offsets are recomputed per issue (they
  // would otherwise hold a register per instruction for the whole kernel).
  auto issue_v = [&](int row0) {
    constexpr int CH = 16 / (int)sizeof(T), CPR = C::LD / CH, NINSTR = kDecWaveKeys * CPR / 64;
    const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vbase + (size_t)row0 * D, min(max(L - row0, 0), kDecWaveKeys) * D);
    // An opaque copy of the lane index keeps the offsets from being hoisted out of the
    // chunk loop, where they would stay live (and spill) for the whole kernel.
    int ln;
    asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
#pragma unroll
    for (int m = 0; m < NINSTR; ++m) {
      const int ch = m * 64 + ln, r = ch / CPR, j = ch - r * CPR;
      dma16_to_lds(vr, sVw + m * 64 * CH, j < D / CH ? (r * D + j * CH) * (int)sizeof(T) : 0x40000000);
    }
  };

  V8 kf[2][C::KS];
  load_k_tile(kf[0], c_last, 0);
  load_k_tile(kf[1], c_last, 1);
  issue_v(c_last * kDecodeChunkKeys + wave * kDecWaveKeys);

  // Q^T fragments: lane l holds query head l%32 of the group (zero past G).
  V8 qf[C::KS];
  {
    const T* qrow = static_cast<const T*>(a.q) + (bh0 + hsafe) * D + hh * 8;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) qf[ks] = head_ok ? ld_vec8(qrow + ks * 16) : zero_vec8<T>();
  }

  // Running state of this wavefront for the lane's head: maximum, sum, O (rows = heads).
  float m_run = kNegInf, l_run = 0.f, carry = 0.f;  // carry: sigma of the keys after this chunk
  f32x16 oacc[C::DT];
#pragma unroll
  for (int j = 0; j < C::DT; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[j][r] = 0.f;

  int par = 0;
  for (int c = c_last; c >= c_first; --c) {
    const int row0 = c * kDecodeChunkKeys + wave * kDecWaveKeys;
    const bool more = c > c_first;

    f32x16 sacc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[i][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) sacc[i] = M::k16(kf[i][ks], qf[ks], sacc[i]);
    }
    // The K fragments are consumed: the next chunk's load into them while this one finishes
    // (tile 0 now, tile 1 before P V, which keeps 32 fewer registers live meanwhile).
    if (kPrefetch && more) load_k_tile(kf[0], c - 1, 0);

    // Scores and sigma.  Key order over the lanes: tile 0 half 0, tile 0 half 1, tile 1
    // half 0, tile 1 half 1.  Keys past L get t = -inf: their sigma is 0 and their a and
    // p follow as -inf and 0 without further masks.
    // Sigma is summed here and recomputed in the suffix pass below rather than kept: the
    // 32 registers it would hold are what keeps this kernel free of spills.
    const int nvalid = L - (row0 + 16 * hh);  // register r of tile i is a key iff 32*i + r < nvalid
    float tot[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[i][r] = 32 * i + r < nvalid ? sacc[i][r] * a.sc2 : kNegInf;
        tot[i] += sigmoid_log2(sacc[i][r]);
        asm volatile("" : "+v"(sacc[i][r]));  // opaque: the compiler would otherwise keep sigma live
      }
    const float oth0 = other_half(tot[0]), oth1 = other_half(tot[1]);
    const float tile1 = tot[1] + oth1;
    if (hh == 0 && head_ok) sSig[par][wave][hl] = tot[0] + oth0 + tile1;
    __syncthreads();
    // z offset of this wavefront: the keys of later wavefronts of the chunk, then of later chunks.
    float off = carry;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float sw = sSig[par][w][hsafe];
      off += w > wave ? sw : 0.f;
      carry += sw;
    }
    par ^= 1;

    float mx = kNegInf;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float z = off + (hh == 0 ? (i == 0 ? oth0 : oth1) : 0.f) + (i == 0 ? tile1 : 0.f);
#pragma unroll
      for (int r = 15; r >= 0; --r) {
        z += sigmoid_log2(sacc[i][r]);
        sacc[i][r] -= lam2 * z;  // a; -inf stays -inf
        mx = fmaxf(mx, sacc[i][r]);
      }
    }
    mx = fmaxf(mx, other_half(mx));
    const float m_new = fmaxf(m_run, mx);
    // Reference point of the exponentials: the running maximum, or 0 while the wavefront
    // has seen no key (then every a is -inf and every weight 0).
    const float mref = m_new == kNegInf ? 0.f : m_new;
    const float fold = fast_exp2(m_run - mref);  // rescale of the running sum / O
    m_run = m_new;

    float lsum = 0.f;
    V8 pa[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x8 pf;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * s + e;
          const float p = fast_exp2(sacc[i][r] - mref);
          pf[e] = p;
          lsum += p;
        }
        pa[i][s] = M::pack(pf);
      }
    l_run = l_run * fold + lsum + other_half(lsum);
    // O rows are query heads: register r of lane l holds head (r/4)*8 + (l/32)*4 + r%4.  The
    // factors go through this wavefront's LDS row (in-order LDS access within a wavefront).
    if (hh == 0) sFold[wave][hl] = fold;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 f = *reinterpret_cast<const f32x4*>(&sFold[wave][g * 8 + hh * 4]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < C::DT; ++j) oacc[j][4 * g + e] *= f[e];
    }

    // V of this chunk has landed once at most the next chunk's K loads are outstanding.
    if (kPrefetch && more) {
      load_k_tile(kf[1], c - 1, 1);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kKLoads));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
#pragma unroll
    for (int j = 0; j < C::DT; ++j)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          oacc[j] = M::k16(pa[i][s], ld_kmajor_dec<T>(sVw, C::LD, 32 * i + 8 * s, 16, 32 * j, lane), oacc[j]);

    if (more) {
      if constexpr (!kPrefetch) {
        load_k_tile(kf[0], c - 1, 0);
        load_k_tile(kf[1], c - 1, 1);
      }
      issue_v(row0 - kDecodeChunkKeys);
    }
  }

  // Combine the wavefronts (their maxima share one z frame: the split's own keys).
  if (hh == 0 && head_ok) {
    sMax[wave][hl] = m_run;
    sSum[wave][hl] = l_run;
  }
  __syncthreads();
  if (tid < G) {
    const int h = tid;
    float m = kNegInf;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) m = fmaxf(m, sMax[w][h]);
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float f = sMax[w][h] == kNegInf ? 0.f : fast_exp2(sMax[w][h] - m);
      sScale[w][h] = f;
      l += f * sSum[w][h];
    }
    const size_t pi = (bh0 + h) * nS + split;
    a.pmax[pi] = m;  // finite: the split's first key is below this sequence's length
    a.psum[pi] = l;
    a.psig[pi] = carry;
  }
  __syncthreads();  // sScale ready; every wavefront is done reading its V tile

  // Scaled O rows (query heads < G) into this wavefront's V region, then summed.
  float* const sO = reinterpret_cast<float*>(sVw);
#pragma unroll
  for (int j = 0; j < C::DT; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int h = (r >> 2) * 8 + hh * 4 + (r & 3);
      if (h < G) sO[h * D + 32 * j + hl] = oacc[j][r] * sScale[wave][h];
    }
  __syncthreads();
  for (int i = tid; i < G * D; i += kDecWaves * 64) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) s += reinterpret_cast<const float*>(sV + w * C::WAVE_ELEMS)[i];
    const int h = i / D, d = i - h * D;
    a.pout[((bh0 + h) * nS + split) * D + d] = s;
  }
}

__device__ __forceinline__ float wave_suffix_sum(float x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_down(x, off, 64);
    if (lane + off < 64) x += y;
  }
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// O and LSE of one (batch, query head) from its split partials.
template <typename T, int D>
__global__ __launch_bounds__(kDecMergeThreads) void coalibi_decode_merge_kernel(DecodeArgs a) {
  constexpr int NW = kDecMergeThreads / 64;
  constexpr int PARTS = kDecMergeThreads / D;
  __shared__ float sW[kMaxDecodeChunks];  // shifted split maxima, then split weights
  __shared__ float sRed[NW];
  __shared__ float sAcc[PARTS][D];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t bh = blockIdx.x;
  const int nS = a.nSplits;
  const float lam2 = a.slopes[bh % a.Hq] * kLog2e;
  const float* pmax = a.pmax + bh * nS;
  const float* psum = a.psum + bh * nS;
  const float* psig = a.psig + bh * nS;

  // Exclusive suffix sums of the split sigma totals, 256 splits at a time from the end; the
  // maximum of split s moves by -slope*log2(e) times the sigma of every later split.
  float carry = 0.f, mx = kNegInf;
  for (int base = (nS - 1) / kDecMergeThreads * kDecMergeThreads; base >= 0; base -= kDecMergeThreads) {
    const int c = base + tid;
    const bool ok = c < nS;
    const float x = ok ? psig[c] : 0.f;
    const float pm = ok ? pmax[c] : 0.f;
    const float suf = wave_suffix_sum(x, lane);
    if (lane == 0) sRed[wave] = suf;
    __syncthreads();
    float later = 0.f, all = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      later += w > wave ? sRed[w] : 0.f;
      all += sRed[w];
    }
    if (ok) {
      const float m = pm - lam2 * (carry + later + suf - x);
      sW[c] = m;
      mx = fmaxf(mx, m);
    }
    carry += all;
    __syncthreads();
  }
  mx = wave_max(mx);
  if (lane == 0) sRed[wave] = mx;
  __syncthreads();
  float m = kNegInf;
#pragma unroll
  for (int w = 0; w < NW; ++w) m = fmaxf(m, sRed[w]);
  __syncthreads();
  // Empty splits (past a sequence's length) have maximum -inf and weight 0; a sequence
  // of length 0 has no split with a key: O = 0 and LSE = -inf.
  const float mref = m == kNegInf ? 0.f : m;
  float l = 0.f;
  for (int c = tid; c < nS; c += kDecMergeThreads) {
    const float w = fast_exp2(sW[c] - mref);
    sW[c] = w;
    l += w * psum[c];
  }
  l = wave_sum(l);
  if (lane == 0) sRed[wave] = l;
  __syncthreads();
  l = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) l += sRed[w];

  // O: thread (part, d) sums the splits part, part + PARTS, ... with eight loads in flight.
  const int d = tid % D, part = tid / D;
  const float* po = a.pout + bh * nS * D + d;
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.f;
  int c = part;
  for (; c + 7 * PARTS < nS; c += 8 * PARTS) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] = fmaf(sW[c + u * PARTS], po[(size_t)(c + u * PARTS) * D], acc[u]);
  }
  for (; c < nS; c += PARTS) acc[0] = fmaf(sW[c], po[(size_t)c * D], acc[0]);
  sAcc[part][d] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (tid < D) {
    float s = 0.f;
#pragma unroll
    for (int p = 0; p < PARTS; ++p) s += sAcc[p][tid];
    static_cast<T*>(a.o)[bh * D + tid] = static_cast<T>(l > 0.f ? s / l : 0.f);
    if (tid == 0 && a.lse != nullptr) a.lse[bh] = l > 0.f ? (m + log2f(l)) * kLn2 : kNegInf;
  }
}

}  // namespace

template <typename T, int D>
hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((coalibi_decode_split_kernel<T, D>), dim3(a.nSplits, a.B * a.Hkv), dim3(kDecWaves * 64), 0,
                     stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((coalibi_decode_merge_kernel<T, D>), dim3(a.B * a.Hq), dim3(kDecMergeThreads), 0, stream, a);
  return hipGetLastError();
}

#define COALIBI_INST_DEC(T, D) template hipError_t launch_decode<T, D>(const DecodeArgs&, hipStream_t);
COALIBI_INST_DEC(_Float16, 32)
COALIBI_INST_DEC(_Float16, 64)
COALIBI_INST_DEC(_Float16, 128)
COALIBI_INST_DEC(_Float16, 256)
COALIBI_INST_DEC(__bf16, 32)
COALIBI_INST_DEC(__bf16, 64)
COALIBI_INST_DEC(__bf16, 128)
COALIBI_INST_DEC(__bf16, 256)
COALIBI_INST_DEC(float, 32)
COALIBI_INST_DEC(float, 64)
COALIBI_INST_DEC(float, 128)

}  // namespace coalibi
