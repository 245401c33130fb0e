// Co-ALiBi decode on gfx950: one new query per (batch, query head) against a key /
// value cache holding L positions, every one of them visible.  In the reference's
// convention (top-left causal alignment, co_alibi_attn/co_alibi_fwd_kernel.py:80-90)
// this is the op with causal=False and Sq = 1:
//   t_j = sm_scale*log2(e) * q.k_j,   sigma_j = sigmoid(t_j / log2(e)),
//   z_j = sum_{k >= j} sigma_k,       a_j = t_j - slope*log2(e) * z_j,
//   O   = sum_j 2^(a_j - m) v_j / sum_j 2^(a_j - m),   LSE = (m + log2 l) * ln 2.
//
// Decode reads the whole cache once for O(L*D) flops per query head: it is bound by
// HBM bandwidth.  The keys form chunks of 128 (one 32-key tile per wavefront), and
// runs of chunks (splits) go to separate work-groups so that every CU streams a part of
// the cache.  Two kernels run:
//   1. split: per (split, batch, kv head), all query heads of the group at once, chunks
//      from the split's last to its first.  S^T = K_chunk Q^T on MFMA (keys on the
//      accumulator rows, the group's query heads on the columns), z from the sigma
//      suffix inside the split only, the split's softmax partial (max, sum, O = P V on
//      MFMA) and its sigma total.
//   2. merge: per (batch, query head).  The keys after chunk c add the same amount
//      off_c = sum_{c' > c} sigma_total[c'] to z_j of every key of chunk c, which
//      shifts a_j of the whole chunk by -slope*log2(e)*off_c and leaves its sum and
//      O partial unchanged once the maximum is shifted by the same amount.  The
//      merge therefore scans the split sigma totals, shifts the split maxima and
//      combines the partials with the usual rescaling.
// K and V go to per-wavefront LDS tiles by buffer-to-LDS DMA, each issued one chunk ahead
// as soon as its tile has been read; K is read back as the MFMA A operand, V as the k-major
// B operand of P V.
#include "coalibi_common.h"
#include "coalibi_kernels.h"

namespace coalibi {

namespace {

constexpr int kDecWaves = 4;
constexpr int kDecWaveKeys = 32;  // keys per wavefront: one 32-key MFMA tile
constexpr int kDecMergeThreads = 256;
static_assert(kDecWaves * kDecWaveKeys == kDecodeChunkKeys, "chunk = the work-group's keys");

template <typename T, int D>
struct DecCfg {
  static constexpr bool kTr = sizeof(T) == 2;
  static constexpr int CH = 16 / (int)sizeof(T);
  // LDS row strides (elements).  K rows are read as MFMA A operands with 16-byte row reads,
  // which a stride of 4 (mod 8) dwords keeps on distinct banks within a read pass.  V rows
  // are read k-major: 16-bit transpose reads (4 rows x 64 bytes a pass) are conflict-free at
  // a stride of 16 (mod 32) dwords; fp32 reads V element by element.
  static constexpr int LDK = D + CH;
  static constexpr int LDV = kTr ? D + 2 * ((48 - (D / 2) % 32) % 32) : D + CH;
  using KTile = DmaTile<T, D, kDecWaveKeys, LDK, 1, true>;
  using VTile = DmaTile<T, D, kDecWaveKeys, LDV, 1, false>;
  static constexpr int K_ELEMS = KTile::LDS_ELEMS;  // a wavefront's K tile
  static constexpr int V_ELEMS = VTile::LDS_ELEMS;  // a wavefront's V tile
  static constexpr int KS = D / 16;  // k16 steps over the head dim
  static constexpr int DT = D / 32;  // 32-column tiles of O
  // At the end the O partials of heads 0..15 alias a wavefront's K tile, of heads 16..31 its V tile.
  static_assert(kMaxDecodeGroup / 2 * D * 4 <= K_ELEMS * (int)sizeof(T) &&
                    kMaxDecodeGroup / 2 * D * 4 <= V_ELEMS * (int)sizeof(T),
                "O partials alias the tiles");
};

// Buffer-to-LDS DMA of the kDecWaveKeys rows row0.. of a row-major [nrows][D] matrix into
// one wavefront's tile (the layout of DmaTile<T, D, kDecWaveKeys, LD, 1, PERM>): every
// instruction reads 64 consecutive 16-byte chunks, non-temporal (the cache is read once per
// step).  Rows past nrows, pad chunks and the tail after the last row land as zeros.  The source offsets are recomputed from an opaque
// copy of the lane index at every issue; hoisted out of the chunk loop they would hold a
// register per instruction for the whole kernel.
template <typename T, int D, int LD, bool PERM>
__device__ __forceinline__ void dma_wave_rows(const T* base, int row0, int nrows, T* lds, int lane) {
  using Tile = DmaTile<T, D, kDecWaveKeys, LD, 1, PERM>;
  const __amdgpu_buffer_rsrc_t r = tile_rsrc(base + (size_t)row0 * D, min(max(nrows - row0, 0), kDecWaveKeys) * D);
  int ln;
  asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
#pragma unroll
  for (int m = 0; m < Tile::NINSTR; ++m) {
    const int ch = m * 64 + ln, row = ch / Tile::CPR, j = ch - row * Tile::CPR;
    const int src = PERM ? (row & ~31) + kRowOfReg(row & 31) : row;
    const bool in_tile = row < kDecWaveKeys && j < D / Tile::CH;
    dma16_to_lds_nt(r, lds + m * 64 * Tile::CH, in_tile ? (src * D + j * Tile::CH) * (int)sizeof(T) : 0x40000000);
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

// The KS fragments (16 bytes each, 32 bytes apart) of one K row of a 16-bit tile, read by
// inline assembly, four per statement, each statement waiting for its own reads before its
// results are used.  Compiled LDS reads of the tile would make the compiler wait, before
// them, for every buffer-to-LDS DMA in flight, the V tile's included; the explicit vmcnt
// waits of the chunk loop already order these reads after the K tile's DMA.
template <typename T, int KS>
__device__ __forceinline__ void ld_k_fragments(typename Mfma<T>::vec8 (&f)[KS], const T* row) {
  static_assert(sizeof(T) == 2 && KS % 2 == 0, "16-bit tiles, an even number of fragments");
  const unsigned a = (unsigned)(size_t)(const __attribute__((address_space(3))) T*)row;  // LDS byte address
  u32x4 u[KS];
#pragma unroll
  for (int g = 0; g + 4 <= KS; g += 4)
    asm volatile(
        "ds_read_b128 %0, %4 offset:%5\n\t"
        "ds_read_b128 %1, %4 offset:%6\n\t"
        "ds_read_b128 %2, %4 offset:%7\n\t"
        "ds_read_b128 %3, %4 offset:%8\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(u[g]), "=&v"(u[g + 1]), "=&v"(u[g + 2]), "=&v"(u[g + 3])
        : "v"(a), "i"(32 * g), "i"(32 * (g + 1)), "i"(32 * (g + 2)), "i"(32 * (g + 3))
        : "memory");
  if constexpr (KS % 4 == 2)
    asm volatile(
        "ds_read_b128 %0, %2 offset:%3\n\t"
        "ds_read_b128 %1, %2 offset:%4\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(u[KS - 2]), "=&v"(u[KS - 1])
        : "v"(a), "i"(32 * (KS - 2)), "i"(32 * (KS - 1))
        : "memory");
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) f[ks] = __builtin_bit_cast(typename Mfma<T>::vec8, u[ks]);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt
// 11:8): at most n vector-memory operations outstanding, or no LDS operation outstanding.
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kLgkmcnt0 = 15 | (3 << 14) | (7 << 4);

template <typename T, int D>
__global__ __launch_bounds__(kDecWaves * 64, (D > 128 || sizeof(T) == 4) ? 1 : 2) void coalibi_decode_split_kernel(
    DecodeArgs a) {
  using M = Mfma<T>;
  using V8 = typename M::vec8;
  using C = DecCfg<T, D>;
  // K tiles, V tiles and the exchange arrays are separate objects: the compiler then knows
  // that reading one does not race the DMA into another, and adds no wait for it.
  __shared__ __align__(16) T sK[kDecWaves * C::K_ELEMS];
  __shared__ __align__(16) T sV[kDecWaves * C::V_ELEMS];
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
  T* const sKw = sK + wave * C::K_ELEMS;  // this wavefront's tiles
  T* const sVw = sV + wave * C::V_ELEMS;
  const bool head_ok = hl < G;
  const int hsafe = head_ok ? hl : 0;
  const float lam2 = a.slopes[hq0 + hsafe] * kLog2e;

  // Both tiles of a chunk come in by DMA (whole 16-byte chunks of consecutive rows: per-lane
  // fragment loads straight from HBM touch 32 rows per instruction and stream at about half
  // the rate).  K rows are permuted (LDS row R holds key kRowOfReg(R)) so that register r of
  // lane l of S^T holds key 16*(l/32) + r of the wavefront.
  auto issue_k = [&](int c) {
    dma_wave_rows<T, D, C::LDK, true>(kbase, c * kDecodeChunkKeys + wave * kDecWaveKeys, L, sKw, lane);
  };
  auto issue_v = [&](int c) {
    dma_wave_rows<T, D, C::LDV, false>(vbase, c * kDecodeChunkKeys + wave * kDecWaveKeys, L, sVw, lane);
  };
  issue_k(c_last);
  issue_v(c_last);

  // Q^T fragments: lane l holds query head l%32 of the group (zero past G).
  V8 qf[C::KS];
  {
    const T* qrow = static_cast<const T*>(a.q) + (bh0 + hsafe) * D + hh * 8;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) qf[ks] = head_ok ? ld_vec8(qrow + ks * 16) : zero_vec8<T>();
  }
  // Wait for Q here, with the first chunk's tiles: the compiler would otherwise place this
  // wait at its first use, inside the chunk loop, as a vmcnt(0) run on every chunk.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

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

    // This chunk's K has landed once at most its V (issued after it) is outstanding.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::VTile::NINSTR));
    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
    if constexpr (C::kTr) {
      V8 kf[C::KS];
      ld_k_fragments<T, C::KS>(kf, sKw + hl * C::LDK + hh * 8);
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) sacc = M::k16(kf[ks], qf[ks], sacc);
    } else {
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) sacc = M::k16(ld_vec8(sKw + hl * C::LDK + ks * 16 + hh * 8), qf[ks], sacc);
    }
    // The K tile has been read: the next chunk's K lands in it during this chunk's math.
    if (more) {
      __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
      issue_k(c - 1);
    }

    // Scores and sigma.  Keys past L get t = -inf: their sigma is 0 and their a and p
    // follow as -inf and 0 without further masks.  Sigma is summed here and recomputed in
    // the suffix pass below rather than kept in registers.
    const int nvalid = L - (row0 + 16 * hh);  // register r is a key iff r < nvalid
    float tot = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = r < nvalid ? sacc[r] * a.sc2 : kNegInf;
      tot += sigmoid_log2(sacc[r]);
      asm volatile("" : "+v"(sacc[r]));  // opaque: the compiler would otherwise keep sigma live
    }
    const float oth = other_half(tot);
    if (hh == 0 && head_ok) sSig[par][wave][hl] = tot + oth;
    lds_barrier();  // the DMA of the next chunk's K stays in flight
    // z offset of this wavefront: the keys of later wavefronts of the chunk, then of later chunks.
    float off = carry;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float sw = sSig[par][w][hsafe];
      off += w > wave ? sw : 0.f;
      carry += sw;
    }
    par ^= 1;

    // Suffix inside the tile: the lower half-wave's keys also see the upper half's total.
    float mx = kNegInf;
    {
      float z = off + (hh == 0 ? oth : 0.f);
#pragma unroll
      for (int r = 15; r >= 0; --r) {
        z += sigmoid_log2(sacc[r]);
        sacc[r] -= lam2 * z;  // a; -inf stays -inf
        mx = fmaxf(mx, sacc[r]);
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
    V8 pa[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      f32x8 pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = fast_exp2(sacc[8 * s + e] - mref);
        pf[e] = p;
        lsum += p;
      }
      pa[s] = M::pack(pf);
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

    // This chunk's V has landed once at most the next chunk's K is outstanding.
    if (more)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::KTile::NINSTR));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    // O^T rows (heads) += P V: B operand rows are keys 8*s + 16*(l/32) + e, as in pa[s].
#pragma unroll
    for (int j = 0; j < C::DT; ++j)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        oacc[j] = M::k16(pa[s], ld_kmajor_dec<T>(sVw, C::LDV, 8 * s, 16, 32 * j, lane), oacc[j]);
    if (more) {
      __builtin_amdgcn_s_waitcnt(kLgkmcnt0);  // the V tile has been read
      issue_v(c - 1);
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
  __syncthreads();  // sScale ready; every wavefront is done with its tiles (no DMA in flight)

  // Scaled O rows (query heads < G) into this wavefront's tiles (heads 0..15 the K tile,
  // 16..31 the V tile), then summed over the wavefronts.
  auto o_row = [&](int w, int h) {
    return reinterpret_cast<float*>(h < kMaxDecodeGroup / 2 ? sK + w * C::K_ELEMS : sV + w * C::V_ELEMS) +
           (h % (kMaxDecodeGroup / 2)) * D;
  };
#pragma unroll
  for (int j = 0; j < C::DT; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int h = (r >> 2) * 8 + hh * 4 + (r & 3);
      if (h < G) o_row(wave, h)[32 * j + hl] = oacc[j][r] * sScale[wave][h];
    }
  __syncthreads();
  for (int i = tid; i < G * D; i += kDecWaves * 64) {
    const int h = i / D, d = i - h * D;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) s += o_row(w, h)[d];
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
  __shared__ float sW[kMaxDecodeSplits];  // shifted split maxima, then split weights
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
