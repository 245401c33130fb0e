// C ABI entry points: argument checks, dtype / head-dim dispatch, launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/co_alibi.h"
#include "coalibi_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t num_zblocks(int seq_kv) { return (static_cast<size_t>(seq_kv) + 31) / 32; }

// fp32 elements of one per-32-key-block array of the recompute path's workspace (zb or cb).
size_t block_sums_numel(int batch, int heads_q, int seq_q, int seq_kv) {
  return static_cast<size_t>(batch) * heads_q * num_zblocks(seq_kv) * seq_q;
}

// The tail skip (the library setting of co_alibi_set_tail_skip): on unless switched off.
std::atomic<int> g_tail_skip{1};

// Where the parts of the forward's statistics lie (coalibi_kernels.h).
struct StatsLayout {
  size_t kstart, knorm, row_order, key_order, rsum, total;  // offsets in 4-byte words
};
StatsLayout stats_layout(int batch, int heads_q, int seq_q, int seq_kv) {
  const size_t bh = static_cast<size_t>(batch) * heads_q;
  StatsLayout l;
  l.kstart = coalibi::kStatsHeader;
  l.knorm = l.kstart + bh * coalibi::stats_kstart_count(seq_q);
  l.row_order = l.knorm + bh * coalibi::stats_knorm_count(seq_kv);
  l.key_order = l.row_order + bh * coalibi::stats_kstart_count(seq_q);
  l.rsum = l.key_order + bh * coalibi::stats_key_block_count(seq_kv);
  l.total = l.rsum + 2 * bh * static_cast<size_t>(seq_q);
  return l;
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct Shape {
  int B, Hq, Hkv, Sq, Skv, D;
};

int check_shape(const char* fn, int dtype, const Shape& s) {
  if (dtype != CO_ALIBI_F32 && dtype != CO_ALIBI_F16 && dtype != CO_ALIBI_BF16)
    return fail(CO_ALIBI_EUNSUPPORTED, std::string(fn) + ": dtype must be 0 (fp32), 1 (fp16) or 2 (bf16)");
  if (s.B < 1 || s.Hq < 1 || s.Hkv < 1 || s.Sq < 1 || s.Skv < 1)
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": batch, heads and sequence lengths must be >= 1");
  if (s.Hq % s.Hkv != 0)
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": heads_q must be a multiple of heads_kv");
  if (s.D != 16 && s.D != 32 && s.D != 64 && s.D != 128 && s.D != 256)
    return fail(CO_ALIBI_EUNSUPPORTED,
                std::string(fn) + ": head_dim must be 16, 32, 64, 128 or 256, got " + std::to_string(s.D));
  // Sequence indices are 32-bit in the kernels; grids must fit a 31-bit launch.
  const double wg = std::ceil(s.Sq / 128.0) * s.B * s.Hq;
  if (s.Sq > (1 << 30) || s.Skv > (1 << 30) || wg > 2147483647.0)
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": problem too large for one launch");
  return CO_ALIBI_OK;
}

// Optional outputs may be NULL; when given they must be aligned.
int check_opt_ptr(const char* fn, const char* name, const void* p, uintptr_t align) {
  if (p != nullptr && !aligned(p, align))
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": " + name + " is not " + std::to_string(align) + "-byte aligned");
  return CO_ALIBI_OK;
}

int check_ptr(const char* fn, const char* name, const void* p, uintptr_t align) {
  if (p == nullptr) return fail(CO_ALIBI_EINVAL, std::string(fn) + ": " + name + " is NULL");
  if (!aligned(p, align))
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": " + name + " is not " + std::to_string(align) + "-byte aligned");
  return CO_ALIBI_OK;
}

template <typename T, int D>
hipError_t fwd_dispatch_causal(const coalibi::FwdArgs& a, bool causal, hipStream_t st) {
  return causal ? coalibi::launch_fwd<T, D, true>(a, st) : coalibi::launch_fwd<T, D, false>(a, st);
}

template <typename T>
hipError_t fwd_dispatch_d(const coalibi::FwdArgs& a, int D, bool causal, hipStream_t st) {
  switch (D) {
    case 16: return fwd_dispatch_causal<T, 16>(a, causal, st);
    case 32: return fwd_dispatch_causal<T, 32>(a, causal, st);
    case 64: return fwd_dispatch_causal<T, 64>(a, causal, st);
    case 256: return fwd_dispatch_causal<T, 256>(a, causal, st);
    default: return fwd_dispatch_causal<T, 128>(a, causal, st);
  }
}

template <typename T, int D>
hipError_t bwd_dispatch_causal(const coalibi::BwdArgs& a, bool causal, int stages, hipStream_t st) {
  return causal ? coalibi::launch_bwd<T, D, true>(a, stages, st) : coalibi::launch_bwd<T, D, false>(a, stages, st);
}

template <typename T>
hipError_t bwd_dispatch_d(const coalibi::BwdArgs& a, int D, bool causal, int stages, hipStream_t st) {
  switch (D) {
    case 16: return bwd_dispatch_causal<T, 16>(a, causal, stages, st);
    case 32: return bwd_dispatch_causal<T, 32>(a, causal, stages, st);
    case 64: return bwd_dispatch_causal<T, 64>(a, causal, stages, st);
    case 256: return bwd_dispatch_causal<T, 256>(a, causal, stages, st);
    default: return bwd_dispatch_causal<T, 128>(a, causal, stages, st);
  }
}

}  // namespace

extern "C" {

size_t co_alibi_stats_numel(int batch, int heads_q, int seq_q, int seq_kv) {
  if (batch < 1 || heads_q < 1 || seq_q < 1 || seq_kv < 1) return 0;
  return stats_layout(batch, heads_q, seq_q, seq_kv).total;
}

size_t co_alibi_bwd_workspace_bytes(int batch, int heads_q, int seq_q, int seq_kv) {
  if (batch < 1 || heads_q < 1 || seq_q < 1 || seq_kv < 1) return 0;
  const size_t rows = static_cast<size_t>(batch) * heads_q * seq_q;
  return round_up(rows * sizeof(float), 256) +
         2 * round_up(block_sums_numel(batch, heads_q, seq_q, seq_kv) * sizeof(float), 256);
}

int co_alibi_set_tail_skip(int enabled) { return g_tail_skip.exchange(enabled != 0 ? 1 : 0); }

int co_alibi_tail_skip(void) { return g_tail_skip.load(); }

size_t co_alibi_bwd_score_store_workspace_bytes(int dtype, int batch, int heads_q, int heads_kv, int seq_q,
                                                int seq_kv, int head_dim, int causal) {
  if (batch < 1 || heads_q < 1 || heads_kv < 1 || heads_q % heads_kv != 0 || seq_q < 1 || seq_kv < 1) return 0;
  if ((dtype != CO_ALIBI_F16 && dtype != CO_ALIBI_BF16) || (head_dim != 64 && head_dim != 128)) return 0;
  if (!coalibi::score_store_fits(heads_q, heads_kv, seq_q)) return 0;
  const size_t rows = static_cast<size_t>(batch) * heads_q * seq_q;
  return round_up(rows * sizeof(float), 256) + static_cast<size_t>(batch) * heads_q *
                                                   coalibi::score_records_per_head(seq_q, seq_kv, causal != 0) *
                                                   coalibi::kScoreRecordBytes;
}

size_t co_alibi_fwd_inference_workspace_bytes(int batch, int heads_q, int seq_q, int seq_kv) {
  if (batch < 1 || heads_q < 1 || seq_q < 1 || seq_kv < 1) return 0;
  return round_up(static_cast<size_t>(batch) * heads_q *
                      (coalibi::stats_knorm_count(seq_kv) + coalibi::stats_kstart_count(seq_q)) * sizeof(float),
                  256);
}

}  // extern "C"

namespace {

// The forward with its statistics (lse and stats: kstart, the key norms and the work orders),
// without them (lse = stats = NULL: no tail skip), or for inference (knorm scratch only: the
// tail skip without the backward's statistics).  With the tail skip switched off
// (co_alibi_set_tail_skip) no key norms are computed and every key is processed.
int fwd_impl(const char* fn, int dtype, const void* q, const void* k, const void* v, const float* slopes, void* o,
             float* lse, float* stats, float* knorm_ws, int batch, int heads_q, int heads_kv, int seq_q,
             int seq_kv, int head_dim, int causal, float sm_scale, void* stream) {
  const Shape s{batch, heads_q, heads_kv, seq_q, seq_kv, head_dim};
  int rc;
  if ((rc = check_shape(fn, dtype, s))) return rc;
  if ((rc = check_ptr(fn, "q", q, 16)) || (rc = check_ptr(fn, "k", k, 16)) || (rc = check_ptr(fn, "v", v, 16)) ||
      (rc = check_ptr(fn, "o", o, 16)) || (rc = check_ptr(fn, "slopes", slopes, 4)) ||
      (rc = check_opt_ptr(fn, "lse", lse, 4)) || (rc = check_opt_ptr(fn, "stats", stats, 4)))
    return rc;
  if (!std::isfinite(sm_scale)) return fail(CO_ALIBI_EINVAL, std::string(fn) + ": sm_scale must be finite");

  coalibi::FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.slopes = slopes;
  a.o = o;
  a.lse = lse;
  const bool skip = g_tail_skip.load() != 0;
  if (stats != nullptr) {  // header, kstart, knorm and the work orders (coalibi_kernels.h)
    const StatsLayout l = stats_layout(batch, heads_q, seq_q, seq_kv);
    int* words = reinterpret_cast<int*>(stats);
    a.flags = words;
    a.kstart = words + l.kstart;
    a.rsum = stats + l.rsum;
    if (skip) {
      a.knorm = stats + l.knorm;
      a.row_order = words + l.row_order;
      a.key_order = words + l.key_order;
    }
  } else if (knorm_ws != nullptr && skip) {  // inference: the row order follows the norms
    a.knorm = knorm_ws;
    a.row_order = reinterpret_cast<int*>(knorm_ws + static_cast<size_t>(batch) * heads_q *
                                                        coalibi::stats_knorm_count(seq_kv));
  }
  a.B = batch;
  a.Hq = heads_q;
  a.Hkv = heads_kv;
  a.Sq = seq_q;
  a.Skv = seq_kv;
  a.nKC = coalibi::stats_knorm_count(seq_kv);
  a.sc2 = sm_scale * coalibi::kLog2eHost;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (dtype) {
    case CO_ALIBI_F16: e = fwd_dispatch_d<_Float16>(a, head_dim, causal != 0, st); break;
    case CO_ALIBI_BF16: e = fwd_dispatch_d<__bf16>(a, head_dim, causal != 0, st); break;
    default: e = fwd_dispatch_d<float>(a, head_dim, causal != 0, st); break;
  }
  if (e != hipSuccess) return fail(CO_ALIBI_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return CO_ALIBI_OK;
}

}  // namespace

extern "C" {

int co_alibi_fwd(int dtype, const void* q, const void* k, const void* v, const float* slopes, void* o,
                 float* lse, float* stats, int batch, int heads_q, int heads_kv, int seq_q, int seq_kv,
                 int head_dim, int causal, float sm_scale, void* stream) {
  return fwd_impl("co_alibi_fwd", dtype, q, k, v, slopes, o, lse, stats, nullptr, batch, heads_q, heads_kv, seq_q,
                  seq_kv, head_dim, causal, sm_scale, stream);
}

int co_alibi_fwd_inference(int dtype, const void* q, const void* k, const void* v, const float* slopes, void* o,
                           void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv, int seq_q,
                           int seq_kv, int head_dim, int causal, float sm_scale, void* stream) {
  const char* fn = "co_alibi_fwd_inference";
  int rc;
  if ((rc = check_ptr(fn, "workspace", workspace, 256))) return rc;
  const size_t need = co_alibi_fwd_inference_workspace_bytes(batch, heads_q, seq_q, seq_kv);
  if (workspace_bytes < need)
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": workspace of " + std::to_string(workspace_bytes) +
                                     " bytes, need " + std::to_string(need));
  return fwd_impl(fn, dtype, q, k, v, slopes, o, nullptr, nullptr, static_cast<float*>(workspace), batch, heads_q,
                  heads_kv, seq_q, seq_kv, head_dim, causal, sm_scale, stream);
}

}  // extern "C"

namespace {

// stages: 1 = pass 1 (dq, dsum, and zb / cb or the score store), 2 = pass 2 (dk, dv), 3 = both.
int bwd_impl(const char* fn, int stages, int dtype, const void* dout, const void* q, const void* k,
             const void* v, const void* o, const float* lse, const float* stats, const float* slopes, void* dq,
             void* dk, void* dv, void* workspace, size_t workspace_bytes, int batch, int heads_q,
             int heads_kv, int seq_q, int seq_kv, int head_dim, int causal, float sm_scale, void* stream) {
  const Shape s{batch, heads_q, heads_kv, seq_q, seq_kv, head_dim};
  int rc;
  if ((rc = check_shape(fn, dtype, s))) return rc;
  if ((rc = check_ptr(fn, "dout", dout, 16)) || (rc = check_ptr(fn, "q", q, 16)) ||
      (rc = check_ptr(fn, "k", k, 16)) || (rc = check_ptr(fn, "v", v, 16)) ||
      (rc = check_ptr(fn, "lse", lse, 4)) || (rc = check_ptr(fn, "stats", stats, 4)) ||
      (rc = check_ptr(fn, "slopes", slopes, 4)) || (rc = check_ptr(fn, "workspace", workspace, 256)))
    return rc;
  if ((stages & 1) && ((rc = check_ptr(fn, "o", o, 16)) || (rc = check_ptr(fn, "dq", dq, 16)))) return rc;
  if ((stages & 2) && ((rc = check_ptr(fn, "dk", dk, 16)) || (rc = check_ptr(fn, "dv", dv, 16)))) return rc;
  // A workspace that holds the score store selects that path (where it exists).
  const size_t need_store =
      co_alibi_bwd_score_store_workspace_bytes(dtype, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal);
  const bool store = need_store != 0 && workspace_bytes >= need_store;
  const size_t need = co_alibi_bwd_workspace_bytes(batch, heads_q, seq_q, seq_kv);
  if (!store && workspace_bytes < need)
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": workspace of " + std::to_string(workspace_bytes) +
                                     " bytes, need " + std::to_string(need));
  if (!std::isfinite(sm_scale)) return fail(CO_ALIBI_EINVAL, std::string(fn) + ": sm_scale must be finite");

  const size_t rows = static_cast<size_t>(batch) * heads_q * seq_q;
  coalibi::BwdArgs a{};
  a.dout = dout;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.slopes = slopes;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.dsum = static_cast<float*>(workspace);
  char* const after_dsum = static_cast<char*>(workspace) + round_up(rows * sizeof(float), 256);
  if (store) {  // the records follow dsum
    a.scores = after_dsum;
    a.score_head = coalibi::score_records_per_head(seq_q, seq_kv, causal != 0);
  } else {  // zb and cb follow dsum
    a.zb = reinterpret_cast<float*>(after_dsum);
    a.cb = reinterpret_cast<float*>(after_dsum +
                                    round_up(block_sums_numel(batch, heads_q, seq_q, seq_kv) * sizeof(float), 256));
  }
  {  // the forward's statistics: header, kstart, knorm, then the work orders it wrote (the
     // kernels follow a table only where the header's flags say it was written)
    const StatsLayout l = stats_layout(batch, heads_q, seq_q, seq_kv);
    const int* words = reinterpret_cast<const int*>(stats);
    a.flags = words;
    a.kstart = words + l.kstart;
    a.rsum = stats + l.rsum;
    a.row_order = words + l.row_order;
    a.key_order = coalibi::key_order_used(batch, heads_q, heads_kv, seq_kv) ? words + l.key_order : nullptr;
  }
  a.B = batch;
  a.Hq = heads_q;
  a.Hkv = heads_kv;
  a.Sq = seq_q;
  a.Skv = seq_kv;
  a.nZB = static_cast<int>(num_zblocks(seq_kv));
  a.sc2 = sm_scale * coalibi::kLog2eHost;
  a.sm_scale = sm_scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (dtype) {
    case CO_ALIBI_F16: e = bwd_dispatch_d<_Float16>(a, head_dim, causal != 0, stages, st); break;
    case CO_ALIBI_BF16: e = bwd_dispatch_d<__bf16>(a, head_dim, causal != 0, stages, st); break;
    default: e = bwd_dispatch_d<float>(a, head_dim, causal != 0, stages, st); break;
  }
  if (e != hipSuccess) return fail(CO_ALIBI_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return CO_ALIBI_OK;
}

}  // namespace

extern "C" {

int co_alibi_bwd(int dtype, const void* dout, const void* q, const void* k, const void* v, const void* o,
                 const float* lse, const float* stats, const float* slopes, void* dq, void* dk, void* dv,
                 void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv, int seq_q,
                 int seq_kv, int head_dim, int causal, float sm_scale, void* stream) {
  return bwd_impl("co_alibi_bwd", 3, dtype, dout, q, k, v, o, lse, stats, slopes, dq, dk, dv, workspace,
                  workspace_bytes, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal, sm_scale, stream);
}

int co_alibi_bwd_dq(int dtype, const void* dout, const void* q, const void* k, const void* v, const void* o,
                    const float* lse, const float* stats, const float* slopes, void* dq, void* workspace,
                    size_t workspace_bytes, int batch, int heads_q, int heads_kv, int seq_q, int seq_kv,
                    int head_dim, int causal, float sm_scale, void* stream) {
  return bwd_impl("co_alibi_bwd_dq", 1, dtype, dout, q, k, v, o, lse, stats, slopes, dq, nullptr, nullptr,
                  workspace, workspace_bytes, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal,
                  sm_scale, stream);
}

int co_alibi_bwd_dkdv(int dtype, const void* dout, const void* q, const void* k, const void* v,
                      const float* lse, const float* stats, const float* slopes, void* dk, void* dv,
                      void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv,
                      int seq_q, int seq_kv, int head_dim, int causal, float sm_scale, void* stream) {
  return bwd_impl("co_alibi_bwd_dkdv", 2, dtype, dout, q, k, v, nullptr, lse, stats, slopes, nullptr, dk, dv,
                  workspace, workspace_bytes, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal,
                  sm_scale, stream);
}

}  // extern "C"

namespace {

template <typename T>
hipError_t decode_dispatch_d(const coalibi::DecodeArgs& a, int D, hipStream_t st) {
  switch (D) {
    case 32: return coalibi::launch_decode<T, 32>(a, st);
    case 64: return coalibi::launch_decode<T, 64>(a, st);
    case 256:
      if constexpr (sizeof(T) == 2) return coalibi::launch_decode<T, 256>(a, st);
      return hipErrorInvalidValue;
    default: return coalibi::launch_decode<T, 128>(a, st);
  }
}

size_t decode_chunks(int seq_kv) {
  return (static_cast<size_t>(seq_kv) + coalibi::kDecodeChunkKeys - 1) / coalibi::kDecodeChunkKeys;
}

// Upper bound of the split count of a decode over seq_kv keys (one split holds >= 1 chunk).
size_t decode_splits_max(int seq_kv) {
  return std::min(decode_chunks(seq_kv), static_cast<size_t>(coalibi::kMaxDecodeSplits));
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Split count of a decode launch: enough splits to give every CU kDecodeWGsPerCU work-groups
// (each split walks cps consecutive 128-key chunks), at most decode_splits_max.
struct DecodeSplit {
  int nChunks, cps, nSplits;
};
DecodeSplit decode_split(int batch, int heads_kv, int seq_kv) {
  DecodeSplit d{};
  d.nChunks = static_cast<int>(decode_chunks(seq_kv));
  const long long units = static_cast<long long>(batch) * heads_kv;
  const long long want = (static_cast<long long>(coalibi::kDecodeWGsPerCU) * device_cus() + units - 1) / units;
  const int splits = static_cast<int>(std::max(1LL, std::min<long long>(want, decode_splits_max(seq_kv))));
  d.cps = (d.nChunks + splits - 1) / splits;
  d.nSplits = (d.nChunks + d.cps - 1) / d.cps;
  return d;
}

// Bytes of split-K partials for `parts` (batch, query head, split) triples: the maximum, the sum
// and the sigma total (one 256-byte aligned fp32 array each), then head_dim floats of O per part.
size_t decode_partials_bytes(size_t parts, int head_dim) {
  return 3 * round_up(parts * sizeof(float), 256) + parts * head_dim * sizeof(float);
}

// Device scratch of co_alibi_decode_noalloc: the split-K partials of callers that cannot
// allocate.  Each GPU holds its own copy for the life of the process.  Host code never uses
// this name as an address: its device address, per device, comes from hipGetSymbolAddress.
constexpr size_t kDecodeScratchBytes = CO_ALIBI_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

// The device address of `scratch` on the current device, looked up once per device (with that
// device current) and kept.
int scratch_address(const char* fn, void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(CO_ALIBI_ELAUNCH, std::string(fn) + ": no current HIP device");
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(CO_ALIBI_ELAUNCH, std::string(fn) + ": scratch lookup failed: " + hipGetErrorString(e));
    addr[dev] = p;
  }
  *out = addr[dev];
  return CO_ALIBI_OK;
}

// co_alibi_decode and co_alibi_decode_noalloc.  The caller's workspace is laid out for the
// largest split count a decode of seq_kv keys can take (its size depends on the shape only);
// the library's scratch is laid out for this launch's split count, which fits more.
int decode_impl(const char* fn, bool scratch_ws, int dtype, const void* q, const void* k_cache,
                const void* v_cache, const float* slopes, const int* seq_lens, void* o, float* lse,
                void* workspace, size_t workspace_bytes, int batch, int heads_q, int heads_kv, int seq_kv,
                int kv_capacity, int head_dim, float sm_scale, void* stream) {
  const Shape s{batch, heads_q, heads_kv, 1, seq_kv, head_dim};
  int rc;
  if ((rc = check_shape(fn, dtype, s))) return rc;
  // The decode kernels read K in pairs of 16-element fragments; a head dim of 16 is one.  The
  // torch operator co_alibi::decode pads such heads to 32 with zero columns, which changes no
  // product.
  if (head_dim == 16)
    return fail(CO_ALIBI_EUNSUPPORTED, std::string(fn) + ": head_dim 16 has no decode kernel (pad q and the "
                                                         "caches to 32 with zeros)");
  // A wavefront's K and V tiles (32 cache rows each) of fp32 at head dim 256 take 66 KB of LDS,
  // four wavefronts more than a CU has.
  if (head_dim == 256 && dtype == CO_ALIBI_F32)
    return fail(CO_ALIBI_EUNSUPPORTED, std::string(fn) + ": decode at head_dim 256 needs fp16 or bf16");
  if (heads_q / heads_kv > coalibi::kMaxDecodeGroup)
    return fail(CO_ALIBI_EUNSUPPORTED, std::string(fn) + ": at most " + std::to_string(coalibi::kMaxDecodeGroup) +
                                           " query heads per kv head");
  if (kv_capacity < seq_kv) return fail(CO_ALIBI_EINVAL, std::string(fn) + ": kv_capacity is below seq_kv");
  if (decode_chunks(seq_kv) > static_cast<size_t>(coalibi::kMaxDecodeChunks))
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": seq_kv above " +
                                     std::to_string(coalibi::kMaxDecodeChunks * coalibi::kDecodeChunkKeys));
  // The workspace size first: it depends on the shape only, and a decode whose partials do not fit
  // is refused before any pointer is looked at.
  const DecodeSplit sp = decode_split(batch, heads_kv, seq_kv);
  const size_t rows = static_cast<size_t>(batch) * heads_q;
  const size_t parts = rows * (scratch_ws ? static_cast<size_t>(sp.nSplits) : decode_splits_max(seq_kv));
  const size_t need = decode_partials_bytes(parts, head_dim);
  if (workspace_bytes < need) {
    if (scratch_ws)
      return fail(CO_ALIBI_EINVAL, std::string(fn) + ": the split-K partials of this decode need " +
                                       std::to_string(need) + " bytes, above the library scratch of " +
                                       std::to_string(workspace_bytes) + " bytes");
    return fail(CO_ALIBI_EINVAL, std::string(fn) + ": workspace of " + std::to_string(workspace_bytes) +
                                     " bytes, need " + std::to_string(need));
  }
  if ((rc = check_ptr(fn, "q", q, 16)) || (rc = check_ptr(fn, "k_cache", k_cache, 16)) ||
      (rc = check_ptr(fn, "v_cache", v_cache, 16)) || (rc = check_ptr(fn, "o", o, 16)) ||
      (rc = check_ptr(fn, "slopes", slopes, 4)) || (rc = check_opt_ptr(fn, "seq_lens", seq_lens, 4)) ||
      (rc = check_opt_ptr(fn, "lse", lse, 4)) || (rc = check_ptr(fn, "workspace", workspace, 256)))
    return rc;
  if (!std::isfinite(sm_scale)) return fail(CO_ALIBI_EINVAL, std::string(fn) + ": sm_scale must be finite");

  const size_t stat_bytes = round_up(parts * sizeof(float), 256);
  char* ws = static_cast<char*>(workspace);
  coalibi::DecodeArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.slopes = slopes;
  a.o = o;
  a.lse = lse;
  a.pmax = reinterpret_cast<float*>(ws);
  a.psum = reinterpret_cast<float*>(ws + stat_bytes);
  a.psig = reinterpret_cast<float*>(ws + 2 * stat_bytes);
  a.pout = reinterpret_cast<float*>(ws + 3 * stat_bytes);
  a.seq_lens = seq_lens;
  a.B = batch;
  a.Hq = heads_q;
  a.Hkv = heads_kv;
  a.G = heads_q / heads_kv;
  a.L = seq_kv;
  a.cap = kv_capacity;
  a.nChunks = sp.nChunks;
  a.cps = sp.cps;
  a.nSplits = sp.nSplits;
  a.sc2 = sm_scale * coalibi::kLog2eHost;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (dtype) {
    case CO_ALIBI_F16: e = decode_dispatch_d<_Float16>(a, head_dim, st); break;
    case CO_ALIBI_BF16: e = decode_dispatch_d<__bf16>(a, head_dim, st); break;
    default: e = decode_dispatch_d<float>(a, head_dim, st); break;
  }
  if (e != hipSuccess) return fail(CO_ALIBI_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return CO_ALIBI_OK;
}

}  // namespace

extern "C" {

size_t co_alibi_decode_workspace_bytes(int batch, int heads_q, int seq_kv, int head_dim) {
  if (batch < 1 || heads_q < 1 || seq_kv < 1 || head_dim < 1) return 0;
  return decode_partials_bytes(static_cast<size_t>(batch) * heads_q * decode_splits_max(seq_kv), head_dim);
}

int co_alibi_decode(int dtype, const void* q, const void* k_cache, const void* v_cache, const float* slopes,
                    const int* seq_lens, void* o, float* lse, void* workspace, size_t workspace_bytes, int batch,
                    int heads_q, int heads_kv, int seq_kv, int kv_capacity, int head_dim, float sm_scale,
                    void* stream) {
  return decode_impl("co_alibi_decode", false, dtype, q, k_cache, v_cache, slopes, seq_lens, o, lse, workspace,
                     workspace_bytes, batch, heads_q, heads_kv, seq_kv, kv_capacity, head_dim, sm_scale, stream);
}

int co_alibi_decode_noalloc(int dtype, const void* q, const void* k_cache, const void* v_cache,
                            const float* slopes, const int* seq_lens, void* o, float* lse, int batch, int heads_q,
                            int heads_kv, int seq_kv, int kv_capacity, int head_dim, float sm_scale, void* stream) {
  const char* fn = "co_alibi_decode_noalloc";
  void* ws = nullptr;
  if (const int rc = scratch_address(fn, &ws)) return rc;
  return decode_impl(fn, true, dtype, q, k_cache, v_cache, slopes, seq_lens, o, lse, ws, kDecodeScratchBytes, batch,
                     heads_q, heads_kv, seq_kv, kv_capacity, head_dim, sm_scale, stream);
}

const char* co_alibi_last_error(void) { return g_last_error.c_str(); }

int co_alibi_abi_version(void) { return 6; }

}  // extern "C"
