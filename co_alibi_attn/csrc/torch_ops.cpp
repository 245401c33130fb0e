// PyTorch-ROCm operators over the C ABI of libco_alibi (include/co_alibi.h).
//
//   co_alibi::fwd(q, k, v, slopes, causal, sm_scale, with_stats) -> (o, lse, stats)
//   co_alibi::bwd(do, q, k, v, o, lse, stats, slopes, causal, sm_scale) -> (dq, dk, dv)
//   co_alibi::bwd_dq(do, q, k, v, o, lse, stats, slopes, causal, sm_scale) -> dq
//   co_alibi::decode(q, k_cache, v_cache, slopes, seq_lens, max_seq_len, sm_scale, with_lse) -> (o, lse)
//
// They replace the reference's two Triton launches with their buffer set-up
// (co_alibi_attn/co_alibi_attn.py:35-57 and :83-133); decode has no counterpart there.  Each
// kernel runs on the caller's current HIP stream under a device guard of the inputs' device and
// allocates only through torch's caching allocator, so the operators can be captured in a HIP
// graph.  co_alibi::fwd carries its backward as a C++ autograd kernel: dQ alone runs backward
// pass 1 only (co_alibi::bwd_dq); any key / value gradient runs both passes (co_alibi::bwd).
// co_alibi::bwd uses the score store (pass 1 keeps s and dS, pass 2 reduces them) where the
// library has it and its workspace fits: at most CO_ALIBI_SCORE_STORE_LIMIT_MB megabytes (an
// environment variable read once; 16384 by default, 0 turns the store off) and at most half
// of the device memory that is free or cached by torch's allocator at the call.  If allocating
// it fails anyway, the backward takes the recompute path, whose workspace is O(S^2 / 32).
// The shape functions for FakeTensor / meta tracing are registered from Python.
#include <ATen/ATen.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <cstdint>
#include <cstdlib>
#include <tuple>

#include "../../include/co_alibi.h"

namespace {

using at::Tensor;

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return CO_ALIBI_F32;
    case at::kHalf: return CO_ALIBI_F16;
    case at::kBFloat16: return CO_ALIBI_BF16;
    default: TORCH_CHECK_TYPE(false, "co_alibi: q, k, v must be float32, float16 or bfloat16, got ", t);
  }
  return -1;
}

void check(int rc) {
  TORCH_CHECK(rc == CO_ALIBI_OK, "co_alibi_attn: ", co_alibi_last_error(), " (status ", rc, ")");
}

// Contiguous tensor whose data pointer is 16-byte aligned (what the kernels load).
Tensor aligned(const Tensor& t) {
  Tensor c = t.contiguous();
  if (reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 != 0) c = c.clone();
  return c;
}

// fp32 copy of the penalty slopes on the inputs' device (no copy when already so).
Tensor slopes_f32(const Tensor& slopes, const Tensor& like) {
  return slopes.detach().to(like.device(), at::kFloat).contiguous();
}

Tensor empty_stats(const Tensor& q) { return at::empty({0}, q.options().dtype(at::kFloat)); }

int64_t stats_numel(int64_t batch, int64_t heads_q, int64_t seq_q, int64_t seq_kv) {
  return static_cast<int64_t>(co_alibi_stats_numel(static_cast<int>(batch), static_cast<int>(heads_q),
                                                   static_cast<int>(seq_q), static_cast<int>(seq_kv)));
}

hipStream_t current_stream(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

// ---------------------------------------------------------------------------- forward

std::tuple<Tensor, Tensor, Tensor> fwd_hip(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in,
                                           const Tensor& slopes, bool causal, double sm_scale, bool with_stats) {
  const int64_t batch = q_in.size(0), heads_q = q_in.size(1), seq_q = q_in.size(2), head_dim = q_in.size(3);
  const int64_t heads_kv = k_in.size(1), seq_kv = k_in.size(2);
  if (q_in.numel() == 0 || seq_kv == 0) {
    // Nothing to launch.  Rows that see no key get what the reference's l = 0 gives:
    // O = 0 / (0 + 1e-9) = 0 and LSE = -inf + log(1e-9) = -inf (co_alibi_fwd_kernel.py:115,120).
    Tensor o = at::zeros(q_in.sizes(), q_in.options());
    if (!with_stats) return {o, empty_stats(q_in), empty_stats(q_in)};
    Tensor lse = at::full({batch, heads_q, seq_q}, -std::numeric_limits<float>::infinity(),
                          q_in.options().dtype(at::kFloat));
    return {o, lse, at::zeros({stats_numel(batch, heads_q, seq_q, seq_kv)}, q_in.options().dtype(at::kFloat))};
  }
  c10::hip::HIPGuard guard(q_in.device().index());
  const Tensor q = aligned(q_in), k = aligned(k_in), v = aligned(v_in);
  const Tensor sl = slopes_f32(slopes, q);
  Tensor o = at::empty_like(q);
  Tensor lse = with_stats ? at::empty({batch, heads_q, seq_q}, q.options().dtype(at::kFloat)) : empty_stats(q);
  Tensor stats = with_stats ? at::empty({stats_numel(batch, heads_q, seq_q, seq_kv)}, q.options().dtype(at::kFloat))
                            : empty_stats(q);
  const int code = dtype_code(q.scalar_type());
  if (with_stats) {
    check(co_alibi_fwd(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), sl.data_ptr<float>(), o.data_ptr(),
                       lse.data_ptr<float>(), stats.data_ptr<float>(), batch, heads_q, heads_kv, seq_q, seq_kv, head_dim,
                       causal ? 1 : 0, static_cast<float>(sm_scale), current_stream(q)));
  } else {  // inference: the tail skip with only its key-norm and work-order scratch
    const size_t ws_bytes = co_alibi_fwd_inference_workspace_bytes(batch, heads_q, seq_q, seq_kv);
    Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
    check(co_alibi_fwd_inference(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), sl.data_ptr<float>(), o.data_ptr(),
                                 ws.data_ptr(), ws_bytes, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim,
                                 causal ? 1 : 0, static_cast<float>(sm_scale), current_stream(q)));
  }
  return {o, lse, stats};
}

// --------------------------------------------------------------------------- backward

// Largest workspace co_alibi::bwd takes for the score store (the environment's limit).
size_t score_store_limit() {
  static const size_t limit = [] {
    const char* e = std::getenv("CO_ALIBI_SCORE_STORE_LIMIT_MB");
    const long long mb = e != nullptr && *e != '\0' ? std::atoll(e) : 16384;
    return mb > 0 ? static_cast<size_t>(mb) << 20 : size_t{0};
  }();
  return limit;
}

// Device memory a new allocation can take on the current device: what the driver reports free
// plus what torch's caching allocator holds unused.
size_t device_memory_available() {
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return 0;
  const auto stats = c10::hip::HIPCachingAllocator::getDeviceStats(c10::hip::current_device());
  const size_t agg = static_cast<size_t>(c10::CachingAllocator::StatType::AGGREGATE);
  const int64_t cached = stats.reserved_bytes[agg].current - stats.allocated_bytes[agg].current;
  return free_b + static_cast<size_t>(cached > 0 ? cached : 0);
}

// Shared set-up of both backward operators; stages 1 = pass 1 only (dq), 3 = both passes.
std::tuple<Tensor, Tensor, Tensor> bwd_common(int stages, const Tensor& do_in, const Tensor& q_in, const Tensor& k_in,
                                              const Tensor& v_in, const Tensor& o_in, const Tensor& lse_in,
                                              const Tensor& stats_in, const Tensor& slopes, bool causal,
                                              double sm_scale) {
  const int64_t batch = q_in.size(0), heads_q = q_in.size(1), seq_q = q_in.size(2), head_dim = q_in.size(3);
  const int64_t heads_kv = k_in.size(1), seq_kv = k_in.size(2);
  if (q_in.numel() == 0 || k_in.numel() == 0) {  // no (query, key) pair: every gradient is zero
    return {at::zeros(q_in.sizes(), q_in.options()), at::zeros(k_in.sizes(), k_in.options()),
            at::zeros(v_in.sizes(), v_in.options())};
  }
  c10::hip::HIPGuard guard(q_in.device().index());
  const Tensor q = aligned(q_in), k = aligned(k_in), v = aligned(v_in), o = aligned(o_in);
  const Tensor dout = aligned(do_in.to(q.scalar_type()));
  const Tensor lse = lse_in.contiguous(), stats = stats_in.contiguous();
  const Tensor sl = slopes_f32(slopes, q);
  Tensor dq = at::empty_like(q);
  Tensor dk = stages & 2 ? at::empty_like(k) : Tensor();
  Tensor dv = stages & 2 ? at::empty_like(v) : Tensor();
  const int code = dtype_code(q.scalar_type());
  size_t ws_bytes = co_alibi_bwd_workspace_bytes(batch, heads_q, seq_q, seq_kv);
  Tensor ws;
  if (stages & 2) {
    const size_t store_bytes =
        co_alibi_bwd_score_store_workspace_bytes(code, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal ? 1 : 0);
    if (store_bytes != 0 && store_bytes <= score_store_limit() && store_bytes <= device_memory_available() / 2) {
      try {
        ws = at::empty({static_cast<int64_t>(store_bytes)}, q.options().dtype(at::kByte));
        ws_bytes = store_bytes;
      } catch (const c10::OutOfMemoryError&) {  // the recompute path's smaller workspace below
      }
    }
  }
  if (!ws.defined()) ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const hipStream_t st = current_stream(q);
  if (stages & 2) {
    check(co_alibi_bwd(code, dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                       lse.data_ptr<float>(), stats.data_ptr<float>(), sl.data_ptr<float>(), dq.data_ptr(),
                       dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, batch, heads_q, heads_kv, seq_q,
                       seq_kv, head_dim, causal ? 1 : 0, static_cast<float>(sm_scale), st));
  } else {
    check(co_alibi_bwd_dq(code, dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                          lse.data_ptr<float>(), stats.data_ptr<float>(), sl.data_ptr<float>(), dq.data_ptr(),
                          ws.data_ptr(), ws_bytes, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal ? 1 : 0,
                          static_cast<float>(sm_scale), st));
  }
  return {dq, dk, dv};
}

std::tuple<Tensor, Tensor, Tensor> bwd_hip(const Tensor& dout, const Tensor& q, const Tensor& k, const Tensor& v,
                                           const Tensor& o, const Tensor& lse, const Tensor& stats,
                                           const Tensor& slopes, bool causal, double sm_scale) {
  return bwd_common(3, dout, q, k, v, o, lse, stats, slopes, causal, sm_scale);
}

Tensor bwd_dq_hip(const Tensor& dout, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& o,
                  const Tensor& lse, const Tensor& stats, const Tensor& slopes, bool causal, double sm_scale) {
  return std::get<0>(bwd_common(1, dout, q, k, v, o, lse, stats, slopes, causal, sm_scale));
}

// ----------------------------------------------------------------------------- decode

std::tuple<Tensor, Tensor> decode_hip(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, const Tensor& slopes,
                                      const c10::optional<Tensor>& seq_lens, int64_t max_seq_len, double sm_scale,
                                      bool with_lse) {
  const int64_t batch = q_in.size(0), heads_q = q_in.size(1), head_dim = q_in.size(3);
  const int64_t heads_kv = k_in.size(1), capacity = k_in.size(2);
  if (q_in.numel() == 0) {  // an empty batch
    Tensor o = at::empty(q_in.sizes(), q_in.options());
    Tensor lse = with_lse ? at::empty({batch, heads_q, 1}, q_in.options().dtype(at::kFloat)) : empty_stats(q_in);
    return {o, lse};
  }
  c10::hip::HIPGuard guard(q_in.device().index());
  if (head_dim == 16) {
    // The decode kernels have no head dim of 16: run on heads padded to 32 with zero columns
    // (the products over d are unchanged, the padding columns of O come out zero) and return
    // the first 16 columns.  This copies the caches once per step.
    auto [o32, lse] = decode_hip(at::constant_pad_nd(q_in, {0, 16}), at::constant_pad_nd(k_in, {0, 16}),
                                 at::constant_pad_nd(v_in, {0, 16}), slopes, seq_lens, max_seq_len, sm_scale, with_lse);
    return {o32.narrow(3, 0, 16).contiguous(), lse};
  }
  const Tensor q = aligned(q_in), k = aligned(k_in), v = aligned(v_in);
  Tensor lens;
  if (seq_lens.has_value() && seq_lens->defined()) lens = seq_lens->to(q.device(), at::kInt).contiguous();
  const Tensor sl = slopes_f32(slopes, q);
  Tensor o = at::empty_like(q);
  Tensor lse = with_lse ? at::empty({batch, heads_q, 1}, q.options().dtype(at::kFloat)) : empty_stats(q);
  const size_t ws_bytes = co_alibi_decode_workspace_bytes(batch, heads_q, max_seq_len, head_dim);
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  check(co_alibi_decode(dtype_code(q.scalar_type()), q.data_ptr(), k.data_ptr(), v.data_ptr(), sl.data_ptr<float>(),
                        lens.defined() ? lens.data_ptr<int>() : nullptr, o.data_ptr(),
                        with_lse ? lse.data_ptr<float>() : nullptr, ws.data_ptr(), ws_bytes, batch, heads_q, heads_kv,
                        max_seq_len, capacity, head_dim, static_cast<float>(sm_scale), current_stream(q)));
  return {o, lse};
}

// --------------------------------------------------------------------------- autograd

// The operators called below autograd (the forward kernel) and from the backward.
std::tuple<Tensor, Tensor, Tensor> call_fwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& slopes,
                                            bool causal, double sm_scale, bool with_stats) {
  static const auto op = c10::Dispatcher::singleton().findSchemaOrThrow("co_alibi::fwd", "").typed<decltype(fwd_hip)>();
  return op.call(q, k, v, slopes, causal, sm_scale, with_stats);
}

// Autograd function of co_alibi::fwd (the role of the reference's CoALIBIAttention,
// co_alibi_attn.py:24-135): saves q, k, v, o, lse, stats and the slopes; lse and stats carry no
// gradient; slopes, causal, sm_scale and with_stats get none.
class FwdFunction : public torch::autograd::Function<FwdFunction> {
 public:
  static torch::autograd::variable_list forward(torch::autograd::AutogradContext* ctx, const Tensor& q,
                                                const Tensor& k, const Tensor& v, const Tensor& slopes, bool causal,
                                                double sm_scale, bool with_stats) {
    Tensor o, lse, stats;
    {
      at::AutoDispatchBelowADInplaceOrView below;
      std::tie(o, lse, stats) = call_fwd(q, k, v, slopes, causal, sm_scale, with_stats);
    }
    ctx->save_for_backward({q, k, v, o, lse, stats, slopes});
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["sm_scale"] = sm_scale;
    ctx->saved_data["with_stats"] = with_stats;
    ctx->mark_non_differentiable({lse, stats});
    // lse and stats never get a gradient: without this the engine would fill zero tensors for
    // them before every backward.
    ctx->set_materialize_grads(false);
    return {o, lse, stats};
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    TORCH_CHECK(ctx->saved_data["with_stats"].toBool(),
                "co_alibi::fwd ran with with_stats=False (inference) and has no backward");
    const auto saved = ctx->get_saved_variables();
    const Tensor &q = saved[0], &k = saved[1], &v = saved[2], &o = saved[3], &lse = saved[4],
                 &stats = saved[5], &slopes = saved[6];
    const bool causal = ctx->saved_data["causal"].toBool();
    const double sm_scale = ctx->saved_data["sm_scale"].toDouble();
    const bool need_q = ctx->needs_input_grad(0), need_k = ctx->needs_input_grad(1), need_v = ctx->needs_input_grad(2);
    Tensor dq, dk, dv;
    const Tensor& dout = grads[0];
    if (dout.defined()) {
      if (!need_k && !need_v) {
        static const auto op_dq =
            c10::Dispatcher::singleton().findSchemaOrThrow("co_alibi::bwd_dq", "").typed<decltype(bwd_dq_hip)>();
        if (need_q) dq = op_dq.call(dout, q, k, v, o, lse, stats, slopes, causal, sm_scale);
      } else {
        static const auto op =
            c10::Dispatcher::singleton().findSchemaOrThrow("co_alibi::bwd", "").typed<decltype(bwd_hip)>();
        std::tie(dq, dk, dv) = op.call(dout, q, k, v, o, lse, stats, slopes, causal, sm_scale);
        if (!need_q) dq = Tensor();
        if (!need_k) dk = Tensor();
        if (!need_v) dv = Tensor();
      }
    }
    return {dq, dk, dv, Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

std::tuple<Tensor, Tensor, Tensor> fwd_autograd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& slopes,
                                                bool causal, double sm_scale, bool with_stats) {
  const auto r = FwdFunction::apply(q, k, v, slopes, causal, sm_scale, with_stats);
  return {r[0], r[1], r[2]};
}

}  // namespace

TORCH_LIBRARY(co_alibi, m) {
  m.def("fwd(Tensor q, Tensor k, Tensor v, Tensor slopes, bool causal, float sm_scale, bool with_stats) -> "
        "(Tensor, Tensor, Tensor)");
  m.def("bwd(Tensor do, Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor stats, Tensor slopes, "
        "bool causal, float sm_scale) -> (Tensor, Tensor, Tensor)");
  m.def("bwd_dq(Tensor do, Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor stats, Tensor slopes, "
        "bool causal, float sm_scale) -> Tensor");
  m.def("decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor slopes, Tensor? seq_lens, SymInt max_seq_len, "
        "float sm_scale, bool with_lse) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(co_alibi, CUDA, m) {
  m.impl("fwd", &fwd_hip);
  m.impl("bwd", &bwd_hip);
  m.impl("bwd_dq", &bwd_dq_hip);
  m.impl("decode", &decode_hip);
}

TORCH_LIBRARY_IMPL(co_alibi, Autograd, m) { m.impl("fwd", &fwd_autograd); }
