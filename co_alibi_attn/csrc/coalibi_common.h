// Shared device helpers for the Co-ALiBi gfx950 kernels.
//
// Matrix products run on CDNA4 MFMA 32x32 tiles.  A "k16 step" is one
// 32x32x16 product: each lane supplies 8 consecutive elements of the
// reduction axis for A and for B (lane l: row/col l%32, reduction half l/32).
// fp16/bf16 use one v_mfma_f32_32x32x16_{f16,bf16}; fp32 (the validation
// mode) issues eight v_mfma_f32_32x32x2_f32, one per element, which reduces
// over the same 16 values because the same (lane, element) -> k assignment is
// used for both operands.
//
// Accumulator layout of a 32x32 tile (16 fp32 per lane): register r of lane l
// holds row (r/4)*8 + (l/32)*4 + (r%4), column l%32.  The kernels read the A
// rows through the permutation kRowOfReg below so that register r of lane l
// holds logical row (l/32)*16 + r: every lane then owns 16 consecutive rows,
// which is what makes the key-axis scans of Co-ALiBi register-local.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace coalibi {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

template <typename T> struct Mfma;

template <> struct Mfma<_Float16> {
  using vec8 = f16x8;
  static __device__ __forceinline__ f32x16 k16(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec8 pack(f32x8 x) { return __builtin_convertvector(x, vec8); }
};

template <> struct Mfma<__bf16> {
  using vec8 = bf16x8;
  static __device__ __forceinline__ f32x16 k16(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec8 pack(f32x8 x) { return __builtin_convertvector(x, vec8); }
};

template <> struct Mfma<float> {
  using vec8 = f32x8;
  static __device__ __forceinline__ f32x16 k16(vec8 a, vec8 b, f32x16 c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], c, 0, 0, 0);
    return c;
  }
  static __device__ __forceinline__ vec8 pack(f32x8 x) { return x; }
};

// Logical row held by MFMA row R (0..31) when A rows are permuted so that
// accumulator register r of lane l holds logical row (l/32)*16 + r.
__device__ __forceinline__ constexpr int kRowOfReg(int R) {
  return ((R >> 2) & 1) * 16 + (R >> 3) * 4 + (R & 3);
}
// Inverse: the MFMA row that must hold logical row k (0..31).
__host__ __device__ __forceinline__ constexpr int kRegOfRow(int k) {
  return ((k >> 2) & 3) * 8 + ((k >> 4) & 1) * 4 + (k & 3);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// sigma(p) with t = p*log2(e):  1 / (1 + 2^-t)
__device__ __forceinline__ float sigmoid_log2(float t) { return fast_rcp(1.0f + fast_exp2(-t)); }

// Value held by the lane in the other half of the wavefront (l ^ 32), through
// v_permlane32_swap (a VALU exchange, no LDS round trip).  With both operands x, the
// instruction's first result holds x of lane l - 32 in lanes 32..63 and its second
// result holds x of lane l + 32 in lanes 0..31.
__device__ __forceinline__ float other_half(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

// Word 3 of a gfx9-family buffer resource for raw (stride 0) dword access: 32-bit data
// format, no swizzle.  Loads at offsets >= num_records return zero.
constexpr int kBufferRsrcWord3 = 0x00020000;

// Buffer resource over `elems` elements at `p`.  Both are wave-uniform at every call site;
// readfirstlane states that to the compiler, which otherwise wraps each load in a loop over
// the distinct resource values of the wave.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const T* p, int elems) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(p);
  const unsigned lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a));
  const unsigned hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(a >> 32));
  const int bytes = __builtin_amdgcn_readfirstlane(elems * (int)sizeof(T));
  void* base = reinterpret_cast<void*>((static_cast<unsigned long long>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, bytes, kBufferRsrcWord3);
}

// Eight consecutive elements at byte offset `off` of a buffer resource (zero past its end):
// one 16-byte load for 16-bit types, two for fp32.  No branch, so a run of these loads goes
// out back to back (a conditional load makes the compiler wait for each one before the next).
template <typename V>
__device__ __forceinline__ V buffer_load_vec8(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (sizeof(V) == 16) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  } else {
    static_assert(sizeof(V) == 32, "eight 2- or 4-byte elements");
    struct { u32x4 lo, hi; } two{__builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0),
                                 __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0)};
    return __builtin_bit_cast(V, two);
  }
}

// 16-byte buffer-to-LDS DMA: lane i of the wavefront writes the 16 bytes at byte offset
// `voffset` of the resource to LDS address lds + 16*i (offsets past the resource read as
// zero).  `lds` must be wave-uniform.  A plain function: inside kernel templates the
// builtin does not survive the host compilation pass.
__device__ __forceinline__ void dma16_to_lds(__amdgpu_buffer_rsrc_t rsrc, void* lds, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
}
// The same DMA, issued by inline assembly so that the compiler does not track it.  The
// compiled builtin counts as an LDS store the compiler cannot place, so it makes every later
// LDS read of the wavefront wait for all DMA in flight, including DMA into another buffer;
// with this form the caller orders the accesses itself: an explicit s_waitcnt vmcnt(0) and a
// barrier before any wavefront reads what the DMA wrote, and a barrier after the last read
// of a buffer before DMA into it is issued.  m0 holds the LDS base of the instruction.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// `lds_byte` is the LDS byte address (wave-uniform), as lds_address() gives it.
__device__ __forceinline__ void dma16_to_lds_untracked(__amdgpu_buffer_rsrc_t rsrc, unsigned lds_byte, int voffset) {
  asm volatile(
      "s_nop 4\n\t"
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds_byte), "v"(voffset), "s"(rsrc)
      : "memory", "m0");
}
#pragma clang diagnostic pop
// The LDS byte address of a pointer into LDS, wave-uniform.  The conversion from a generic
// pointer tests it for null (scalar instructions): a loop takes it once, outside.
__device__ __forceinline__ unsigned lds_address(const void* lds) {
  return __builtin_amdgcn_readfirstlane((unsigned)(size_t)(const __attribute__((address_space(3))) void*)lds);
}
// The same with the non-temporal cache policy (the "nt" bit, cache-policy value 2), for data
// read exactly once: a stream of such loads sustains about 15 % more HBM bandwidth on
// MI355X (6.9 against 6.0 TB/s in a read-only test of this access pattern).
constexpr int kCachePolicyNt = 2;
__device__ __forceinline__ void dma16_to_lds_nt(__amdgpu_buffer_rsrc_t rsrc, void* lds, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0,
                                           kCachePolicyNt);
}

// Work-group barrier for data exchanged through LDS by ordinary LDS stores: each wavefront
// waits for its own LDS operations (lgkmcnt) and meets the others.  __syncthreads(), and even
// a fence restricted to LDS, also wait for every vector-memory operation in flight (vmcnt(0),
// which counts buffer-to-LDS DMA as LDS stores); this one lets prefetches and DMA continue, so
// it must not be used to publish DMA-written LDS.  The memory clobber keeps the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16-byte global / LDS accessors.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec8 ld_vec8(const T* p) {
  return *reinterpret_cast<const typename Mfma<T>::vec8*>(p);
}

// x * s, rounded back to T once per element.  The 16-bit kernels fold sm_scale*log2(e)
// into the Q fragments with this, so S^T comes out of the MFMA already in log2 units.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec8 scale_vec8(typename Mfma<T>::vec8 x, float s) {
  f32x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = static_cast<float>(x[e]) * s;
  return Mfma<T>::pack(f);
}

template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec8 zero_vec8() {
  typename Mfma<T>::vec8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = T(0);
  return z;
}

// Work order of a grid of row or key blocks over B*H (batch, head) pairs (H query heads
// for row-block grids, H key heads for key-block grids).  Ids are taken rank-major,
// head-minor, where rank 0 is the block with the most work (the longest causal rows, or
// the key block seen by the most query rows); the dispatcher hands consecutive work-group
// ids to the 8 XCDs in turn, so position j of a rank runs on XCD j mod 8, and every XCD
// sees its blocks in decreasing cost (longest-processing-time-first list scheduling keeps
// the tail short).
//
// Which head sits at position j balances the XCDs.  The tail skip cuts a head's work by
// its slope (a larger slope skips more keys), so heads differ in work by up to 30x, and a
// head kept on one XCD leaves that XCD busy long after the others.  Two orders, chosen by
// same-box measurement per kernel (headline, gqa and long configs):
//   lpt_item: the heads of rank r are rotated by r / rotate positions.  With rotate = 1 the
//     blocks of a head visit the XCDs in turn (the forward and pass 1: each block reads
//     its own Q rows and a key range, so the XCDs' L2 sharing matters little);
//   balanced_item: the heads are ranked by their smallest slope (for a key head, over its
//     query heads; larger first, so lighter first), the (rank, batch) pairs are numbered in
//     that order and dealt to positions in boustrophedon order over the 8 XCDs (0..7,
//     7..0, ...), so each XCD serves a mix of light and heavy heads, and runs of
//     kLptRotateRanks consecutive blocks of a head share an XCD and its L2 (pass 2: the
//     key blocks of a head read the same Q / dO tiles).  Heads beyond kMaxBalancedHeads keep
//     their index order.
constexpr int kLptRotateRanks = 4;
struct WorkItem {
  int head;  // b * H + h
  int rank;  // 0 = most work
};
__device__ __forceinline__ WorkItem lpt_item(int id, int heads, int rotate) {
  const int rank = id / heads;
  return {(id - rank * heads + rank / rotate) % heads, rank};
}
// The item of work-group `id` from a work-order table (coalibi_kernels.h): entry id holds
// rank * heads + head.  The entry is clamped into the grid's items, so a table that is not a
// permutation cannot send a work-group out of bounds.
__device__ __forceinline__ WorkItem table_item(const int* __restrict__ order, int id, int heads, int items) {
  const int i = min(max(order[id], 0), items - 1);
  const int rank = i / heads;
  return {i - rank * heads, rank};
}
constexpr int kMaxBalancedHeads = 256;
// `key` and `order` (kMaxBalancedHeads floats / ints of LDS scratch, free again on return)
// hold the heads' slopes and rank order; every thread of the work-group calls this (three
// barriers).
// `rotate`: ranks per rotation step (kLptRotateRanks; without the tail skip every head has the
// same work, and a rotate past the ranks keeps each head on one XCD).
__device__ __forceinline__ WorkItem balanced_item(int id, int B, int H, const float* __restrict__ slopes,
                                                  int group, float* key, int* order, int tid, int nthreads,
                                                  int rotate) {
  const int heads = B * H;
  const int rank = id / heads;
  int j = id - rank * heads;
  j = (j + rank / rotate) % heads;
  if (H > kMaxBalancedHeads) return {j, rank};
  for (int t = tid; t < H; t += nthreads) {
    float m = __builtin_inff();
    for (int g = 0; g < group; ++g) {
      const float l = slopes[t * group + g];
      m = fminf(m, l > 0.f ? l : 0.f);  // no skip for a slope <= 0 (or NaN): heaviest
    }
    key[t] = m;
  }
  __syncthreads();
  for (int t = tid; t < H; t += nthreads) {
    const float kt = key[t];
    int r = 0;
    for (int u = 0; u < H; ++u) r += (key[u] > kt) || (key[u] == kt && u < t);
    order[r] = t;
  }
  __syncthreads();
  const int blk = j >> 3, x = j & 7;
  const bool whole = (blk + 1) * 8 <= heads;  // a partial last block of 8 keeps its order
  const int n = (whole && (blk & 1)) ? blk * 8 + 7 - x : j;  // number in rank order
  const int h = order[n / B], b = n - (n / B) * B;
  __syncthreads();  // the scratch may be reused once every wavefront has read its head
  return {b * H + h, rank};
}

}  // namespace coalibi

namespace coalibi {

template <typename T, int N> struct VecOf { typedef T type __attribute__((ext_vector_type(N))); };

// A ROWS x D tile of a row-major [nrows][D] matrix staged into an LDS tile of row
// stride LD (elements, padded) by buffer-to-LDS DMA.  One DMA instruction writes 64
// consecutive 16-byte chunks, so the padded tile is a run of ROWS*LD*sizeof(T)/16
// chunks, rounded up to whole instructions (LDS_ELEMS elements: the chunks past the
// tile land in that tail), split over the work-group's NWAVES wavefronts; each lane
// keeps the source offset of its chunk in every instruction slot it issues
// (tile-invariant).  Pad chunks, the tail and rows at or beyond `nrows` point past the
// buffer resource and land as zeros.  PERM: LDS row R of every 32-row block holds
// source row kRowOfReg(R), the order in which an A operand with keys on the
// accumulator rows reads them.
template <typename T, int D, int ROWS, int LD, int NWAVES, bool PERM>
struct DmaTile {
  static constexpr int CH = 16 / (int)sizeof(T);        // elements per 16-byte chunk
  static constexpr int CPR = LD * (int)sizeof(T) / 16;  // chunks per padded LDS row
  static constexpr int NINSTR = (ROWS * CPR + 63) / 64;  // wavefront DMA instructions per tile
  static constexpr int LDS_ELEMS = NINSTR * 64 * CH;     // LDS the tile's instructions write
  static constexpr int SLOTS = (NINSTR + NWAVES - 1) / NWAVES;
  static_assert(NWAVES * (SLOTS - 1) < NINSTR, "every slot but the last holds an instruction");
  static_assert(LD * (int)sizeof(T) % 16 == 0 && LD >= D, "rows must be whole 16-byte chunks");
  static_assert(!PERM || ROWS % 32 == 0, "rows are permuted in blocks of 32");
  int off[SLOTS];

  __device__ __forceinline__ void init(int wave, int lane) {
#pragma unroll
    for (int m = 0; m < SLOTS; ++m) {
      const int c = (wave + NWAVES * m) * 64 + lane;
      const int r = c / CPR, j = c - r * CPR;
      const int src = PERM ? (r & ~31) + kRowOfReg(r & 31) : r;
      off[m] = j < D / CH ? (src * D + j * CH) * (int)sizeof(T) : 0x40000000;
    }
  }
  __device__ __forceinline__ void issue(const T* base, int row0, int nrows, T* lds, int wave) const {
    const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(base + (size_t)row0 * D, min(max(nrows - row0, 0), ROWS) * D);
#pragma unroll
    for (int m = 0; m < SLOTS; ++m) {
      const int i = wave + NWAVES * m;
      if (i < NINSTR) dma16_to_lds(rsrc, lds + i * 64 * 16 / (int)sizeof(T), off[m]);
    }
  }
  // The same through dma16_to_lds_untracked (its rules apply), into the tile at LDS byte
  // address lds_byte (lds_address).  wave < NWAVES, so only the last slot can lie past the
  // tile's instructions.
  __device__ __forceinline__ void issue_untracked(const T* base, int row0, int nrows, unsigned lds_byte,
                                                  int wave) const {
    const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(base + (size_t)row0 * D, min(max(nrows - row0, 0), ROWS) * D);
#pragma unroll
    for (int m = 0; m < SLOTS; ++m) {
      const int i = wave + NWAVES * m;
      if (m + 1 < SLOTS || i < NINSTR) dma16_to_lds_untracked(rsrc, lds_byte + i * 64 * 16, off[m]);
    }
  }
};

// Zero `bytes` (a multiple of 16) of LDS with the whole work-group of `nthreads`.
__device__ __forceinline__ void lds_zero(void* p, int bytes, int tid, int nthreads) {
  u32x4* z = reinterpret_cast<u32x4*>(p);
  for (int i = tid; i < bytes / 16; i += nthreads) z[i] = u32x4{0u, 0u, 0u, 0u};
}

// Stages a ROWS x D tile of a row-major [rows][D] matrix through registers into
// LDS, 16 bytes per load/store.  Rows at or beyond `nrows` read as zero.
//   GROUPED = false: consecutive threads own consecutive 16-byte chunks of a row
//     (coalesced loads, conflict-free row stores); only store_rows is available.
//   GROUPED = true: each thread owns KG consecutive rows x one chunk, so the same
//     registers can also be written transposed (store_cols, the [D][rows] layout
//     used where no transpose read exists, i.e. for fp32).
// store_rows<PERM> writes row-major; with PERM, rows are permuted with kRegOfRow
// inside every 32-row block (the layout the A operand of a "rows along
// registers" product reads in lane order).
template <typename T, int D, int ROWS, bool GROUPED = false>
struct TileLoader {
  static constexpr int CH = 16 / sizeof(T);  // elements per chunk
  static constexpr int CPR = D / CH;         // chunks per row
  // Rows per thread group: the largest of 4, 2, 1 that still gives every thread a group.
  static constexpr int KG = !GROUPED ? 1
                            : ((ROWS / 4) * CPR >= 256) ? 4 : ((ROWS / 2) * CPR >= 256) ? 2 : 1;
  static constexpr int NG = (ROWS / KG) * CPR;  // groups per tile
  static constexpr int GPT = (NG + 255) / 256;  // groups per thread
  static constexpr bool kPartial = NG % 256 != 0;  // small tiles: threads >= NG idle
  static_assert(NG < 256 || NG % 256 == 0, "tile does not split over 256 threads");
  static_assert(ROWS % 32 == 0, "rows are permuted in blocks of 32");

  u32x4 r[GPT][KG];

  __device__ __forceinline__ static int grp_row(int g) { return GROUPED ? (g % (ROWS / KG)) * KG : g / CPR; }
  __device__ __forceinline__ static int grp_col(int g) { return GROUPED ? (g / (ROWS / KG)) * CH : (g % CPR) * CH; }

  // Rows row0 .. row0+ROWS-1 of a row-major [nrows][D] array; rows >= nrows read as zero.
  // Buffer loads: the resource covers exactly the tile's valid rows, so the hardware range
  // check zero-fills the rest; per-lane offsets are tile-invariant and the base is uniform.
  __device__ __forceinline__ void load(const T* __restrict__ base, int row0, int nrows, int tid) {
    const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(base + (size_t)row0 * D, min(max(nrows - row0, 0), ROWS) * D);
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = tid + 256 * i;
      if (kPartial && g >= NG) continue;
      const int rr = grp_row(g), cc = grp_col(g);
#pragma unroll
      for (int k = 0; k < KG; ++k)
        r[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, ((rr + k) * D + cc) * (int)sizeof(T), 0, 0);
    }
  }

  template <bool PERM = true>
  __device__ __forceinline__ void store_rows(T* s, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = tid + 256 * i;
      if (kPartial && g >= NG) continue;
      const int rr = grp_row(g), cc = grp_col(g);
#pragma unroll
      for (int k = 0; k < KG; ++k) {
        const int row = rr + k;
        const int R = PERM ? ((row & ~31) | kRegOfRow(row & 31)) : row;
        st16(s + R * ld + cc, r[i][k]);
      }
    }
  }

  // s[c * ld + row] (rows in natural order)
  __device__ __forceinline__ void store_cols(T* s, int ld, int tid) const {
    static_assert(GROUPED, "store_cols needs the grouped layout");
    using chunk = typename VecOf<T, CH>::type;
    using grp = typename VecOf<T, KG>::type;
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int g = tid + 256 * i;
      if (kPartial && g >= NG) continue;
      const int rr = grp_row(g), cc = grp_col(g);
      chunk rows[KG];
#pragma unroll
      for (int k = 0; k < KG; ++k) rows[k] = __builtin_bit_cast(chunk, r[i][k]);
#pragma unroll
      for (int e = 0; e < CH; ++e) {
        grp w;
#pragma unroll
        for (int k = 0; k < KG; ++k) w[k] = rows[k][e];
        *reinterpret_cast<grp*>(s + (cc + e) * ld + rr) = w;
      }
    }
  }
};

}  // namespace coalibi

namespace coalibi {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __fp16 tr_f16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __bf16 tr_bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));

// Physical LDS row of logical row r in a tile stored with store_rows<true>.
__device__ __forceinline__ int perm_row(int r) { return (r & ~31) | kRegOfRow(r & 31); }

// One ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives
// element j of the 8 bytes addressed by group-lane 4*j + i/4, position i%4.
template <typename T>
__device__ __forceinline__ u32x2 lds_tr4(const T* p) {
  if constexpr (__is_same(T, _Float16)) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                         (__attribute__((address_space(3))) tr_f16x4*)(p)));
  } else {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                         (__attribute__((address_space(3))) tr_bf16x4*)(p)));
  }
}

// MFMA 32x32x16 operand whose reduction index runs along the rows of a
// row-major 16-bit LDS tile: lane l receives tile[row(l/32, e)][col0 + l%32]
// for e = 0..7, with row(kh, e) = rbase + kh*khs + e (through perm_row when
// PERM).  Two transpose reads; each 16-lane group gathers 4 rows x 16 columns.
template <typename T, bool PERM>
__device__ __forceinline__ typename Mfma<T>::vec8 ld_kmajor(const T* tile, int ld, int rbase, int khs,
                                                              int col0, int lane) {
  static_assert(sizeof(T) == 2, "transpose reads are 16-bit only");
  const int i = lane & 15, g = lane >> 4;
  const int col = col0 + 16 * (g & 1) + 4 * (i & 3);
  const int r0 = rbase + (g >> 1) * khs + (i >> 2);
  const int ra = PERM ? perm_row(r0) : r0;
  const int rb = PERM ? perm_row(r0 + 4) : r0 + 4;
  const u32x2 lo = lds_tr4(tile + ra * ld + col);
  const u32x2 hi = lds_tr4(tile + rb * ld + col);
  return __builtin_bit_cast(typename Mfma<T>::vec8, u32x4{lo[0], lo[1], hi[0], hi[1]});
}

// Adds the eight values of a packed operand to an fp32 sum.
__device__ __forceinline__ float sum8(f16x8 v, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2) acc = __builtin_amdgcn_fdot2(h2{v[e], v[e + 1]}, h2{1, 1}, acc, false);
  return acc;
}
__device__ __forceinline__ float sum8(bf16x8 v, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2) acc = __builtin_amdgcn_fdot2_f32_bf16(b2{v[e], v[e + 1]}, b2{1, 1}, acc, false);
  return acc;
}
__device__ __forceinline__ float sum8(f32x8 v, float acc) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc += v[e];
  return acc;
}

}  // namespace coalibi
