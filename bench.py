"""Benchmark of the Co-ALiBi attention hot path on one MI355X.

A step is one forward + backward of ``co_alibi_attention`` over the headline
workload (B=4, Hq=Hkv=16, S=4096, D=128, fp16,
causal, q/k/v ~ 0.5 N(0,1), dO ~ N(0,1), seed 0), inputs resident in HBM.
``value`` is algorithmic TFLOP/s of the step in the FlashAttention convention
(fwd 4*B*H*S^2*D/2 for causal, bwd 2.5x fwd).  Prints one JSON line.

Also measured in the same run:
  * each kernel alone through the C ABI with HIP events on the launch stream
    (forward, backward pass 1, backward pass 2); the longest one is reported
    in ``roofline`` against the dense fp16 MFMA peak;
  * the CPU baseline: the repository's CPU restatement of model.py (oracle,
    fp32) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_PEAK_TFLOPS = {"fp16": 2516.6, "bf16": 2516.6, "fp32": 157.3}  # MI355X dense
HBM_PEAK_GBS = 8000.0


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="headline", choices=["headline", "gqa", "long", "cpu"])
    ap.add_argument("--cpu-heads", type=int, default=16,
                    help="query heads of batch 0 in the CPU-baseline sample (0 disables it)")
    ap.add_argument("--kernel-reps", type=int, default=20, help="launches per kernel in the per-kernel timing")
    return ap.parse_args()


def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(w, heads: int):
    """Times the CPU oracle (fp32 restatement of model.py) on batch 0, query heads [0, heads)."""
    import torch

    from co_alibi_attn.workloads import make_inputs
    from oracle import co_alibi_ref as ref

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    q, k, v, do = (t.float() for t in make_inputs(w, seed=0, batch=1))
    lam = ref.slopes(w.heads_q, w.bias_max, dtype=w.dtype).float()
    g = w.heads_q // w.heads_kv
    pairs = [(0, h) for h in range(min(heads, w.heads_q))]
    scale = 1.0 / math.sqrt(w.head_dim)
    t0 = time.perf_counter()
    ref.forward(q, k, v, lam, causal=w.causal, scale=scale, heads=pairs)
    ref.backward(do, q, k, v, lam, causal=w.causal, scale=scale, heads=pairs)
    secs = time.perf_counter() - t0
    fwd, bwd = ref.flops(1, len(pairs), w.seq, w.seq, w.head_dim, w.causal)
    sample = (f"{w.name} workload, batch 0, query heads 0..{len(pairs) - 1} (of {w.batch}x{w.heads_q}), "
              f"fwd+bwd fp32, {secs:.1f} s on {cores} threads of {cpu_model_name()}")
    del g
    return {"value": (fwd + bwd) / secs / 1e12, "unit": "TFLOPS", "cores": cores, "kind": "port",
            "sample": sample, "seconds": round(secs, 3)}


def cpu_config_timing():
    """BASELINE configs[0] (B1 H2 S128 D64 fp32) fwd+bwd on the CPU oracle: median of 20 after 3 warmups."""
    import torch

    from co_alibi_attn.workloads import WORKLOADS, make_inputs
    from oracle import co_alibi_ref as ref

    w = WORKLOADS["cpu"]
    q, k, v, do = make_inputs(w, seed=0)
    lam = ref.slopes(w.heads_q, w.bias_max, dtype=w.dtype)
    times = []
    for i in range(23):
        t0 = time.perf_counter()
        ref.forward(q, k, v, lam)
        ref.backward(do, q, k, v, lam)
        if i >= 3:
            times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2] * 1e3


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the Co-ALiBi op is single-GPU; sharding is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch

    from co_alibi_attn import _native, co_alibi_attention
    from co_alibi_attn.workloads import WORKLOADS, make_inputs
    from oracle.co_alibi_ref import flops

    w = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    dtype_name = {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[w.dtype]
    q, k, v, do = make_inputs(w, seed=0, device=dev)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    fwd_flops, bwd_flops = flops(w.batch, w.heads_q, w.seq, w.seq, w.head_dim, w.causal)
    print(f"[bench] workload {w.name}: B{w.batch} Hq{w.heads_q} Hkv{w.heads_kv} S{w.seq} D{w.head_dim} "
          f"{dtype_name} causal={w.causal}", file=sys.stderr, flush=True)

    def step():
        q.grad = k.grad = v.grad = None
        o = co_alibi_attention(q, k, v, causal=w.causal, bias_max=w.bias_max)
        o.backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(end) / args.steps
    value = (fwd_flops + bwd_flops) / (ms_step * 1e-3) / 1e12
    print(f"[bench] {args.steps} steps: {ms_step:.3f} ms/step (wall {wall:.2f} s)", file=sys.stderr, flush=True)

    # Per-kernel timing through the C ABI on torch's current stream.
    lib = _native.lib()
    B, Hq, Hkv, S, D = w.batch, w.heads_q, w.heads_kv, w.seq, w.head_dim
    code = _native.DTYPE_CODES[w.dtype]
    from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes

    lam = (2.0 * _get_coalibi_slopes(Hq, w.bias_max)).to(w.dtype).float().to(dev)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd = q.detach(), k.detach(), v.detach()
    o = torch.empty_like(qd)
    lse = torch.empty(B, Hq, S, device=dev, dtype=torch.float32)
    zb = torch.empty(lib.co_alibi_zb_numel(B, Hq, S, S), device=dev, dtype=torch.float32)
    ws_bytes = lib.co_alibi_bwd_workspace_bytes(B, Hq, S, S)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    shape = (B, Hq, Hkv, S, S, D, int(w.causal), scale, sh)

    def k_fwd():
        _native.check(lib.co_alibi_fwd(code, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), lam.data_ptr(),
                                       o.data_ptr(), lse.data_ptr(), zb.data_ptr(), *shape))

    def k_dq():
        _native.check(lib.co_alibi_bwd_dq(code, do.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                          o.data_ptr(), lse.data_ptr(), zb.data_ptr(), lam.data_ptr(),
                                          dq.data_ptr(), ws.data_ptr(), ws_bytes, *shape))

    def k_dkdv():
        _native.check(lib.co_alibi_bwd_dkdv(code, do.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                            lse.data_ptr(), zb.data_ptr(), lam.data_ptr(), dk.data_ptr(),
                                            dv.data_ptr(), ws.data_ptr(), ws_bytes, *shape))

    # Issued GEMM work per launch: fwd 2 products (QK^T, PV); pass 1 three (S, dS, dQ);
    # pass 2 four (S, dS, dV, dK), each 2*B*Hq*D per visible (query, key) pair.
    gemm = fwd_flops / 2.0
    kernels = {"coalibi_fwd_kernel": (k_fwd, 2 * gemm), "coalibi_bwd_dq_kernel": (k_dq, 3 * gemm),
               "coalibi_bwd_dkdv_kernel": (k_dkdv, 4 * gemm)}
    k_fwd()
    k_dq()
    k_dkdv()
    torch.cuda.synchronize()
    per_kernel = {}
    for name, (fn, kflops) in kernels.items():
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.kernel_reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.kernel_reps
        per_kernel[name] = {"ms": round(ms, 4), "tflops": round(kflops / (ms * 1e-3) / 1e12, 2),
                            "issued_gflop": round(kflops / 1e9, 2)}
    fwd_ms = per_kernel["coalibi_fwd_kernel"]["ms"]
    bwd_ms = per_kernel["coalibi_bwd_dq_kernel"]["ms"] + per_kernel["coalibi_bwd_dkdv_kernel"]["ms"]
    dominant = max(per_kernel, key=lambda n: per_kernel[n]["ms"])
    peak = MFMA_PEAK_TFLOPS[dtype_name]
    achieved = per_kernel[dominant]["tflops"]
    print(f"[bench] per-kernel: {json.dumps(per_kernel)}", file=sys.stderr, flush=True)

    out = {
        "metric": "fwd and bwd TFLOPS (and % of MFMA peak) at B4 H16 S4096 D128 fp16 causal",
        "value": round(value, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name,
        "data": "synthetic (seeded N(0,1) inputs of the BASELINE shape)",
        "config": {"workload": f"co_alibi_attention fwd+bwd, {w.name}", "batch": B, "heads_q": Hq,
                   "heads_kv": Hkv, "seq_len": S, "head_dim": D, "causal": w.causal, "bias_max": w.bias_max},
        "fwd_ms": fwd_ms,
        "bwd_ms": round(bwd_ms, 4),
        "fwd_tflops": round(fwd_flops / (fwd_ms * 1e-3) / 1e12, 2),
        "bwd_tflops": round(bwd_flops / (bwd_ms * 1e-3) / 1e12, 2),
        "fwd_frac_peak": round(fwd_flops / (fwd_ms * 1e-3) / 1e12 / peak, 4),
        "bwd_frac_peak": round(bwd_flops / (bwd_ms * 1e-3) / 1e12 / peak, 4),
        "ref_convention_tflops": {"fwd": round(2 * fwd_flops / (fwd_ms * 1e-3) / 1e12, 2),
                                  "bwd": round(4 * fwd_flops / (bwd_ms * 1e-3) / 1e12, 2)},
        "kernels": per_kernel,
        "roofline": {"kernel": dominant, "bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": None},
    }
    if args.cpu_heads > 0:
        print("[bench] CPU baseline ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(w, args.cpu_heads)
        out["cpu_config0_ms"] = round(cpu_config_timing(), 3)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
