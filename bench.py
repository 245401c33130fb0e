"""Benchmark of the Co-ALiBi attention hot path on one MI355X.

A step is one forward + backward of ``co_alibi_attention`` over the headline
workload (B=4, Hq=Hkv=16, S=4096, D=128, fp16,
causal, q/k/v ~ 0.5 N(0,1), dO ~ N(0,1), seed 0), inputs resident in HBM.
``value`` is the step's effective TFLOP/s: algorithmic flops in the FlashAttention
convention (fwd 4*B*H*S^2*D/2 for causal, bwd 2.5x fwd) over the step time, with the
library's tail skip on (its default: keys whose softmax weight is provably negligible
are left out).  Prints one JSON line.

Also measured in the same run:
  * the full-work figures, with the tail skip off (every visible tile processed, as the
    reference's kernels do): ``fwd_frac_peak`` and ``bwd_frac_peak`` are these, algorithmic
    flops over kernel time against the dense fp16 MFMA peak -- the north star's fractions;
  * each kernel alone through the C ABI with HIP events on the launch stream (forward,
    backward pass 1, backward pass 2), skip on and off: its time, effective TFLOP/s, and
    the flops its MFMA units actually issue, counted from the tiles the forward recorded as
    processed (profiling.issued_k16); the longest skip-on kernel is reported in
    ``roofline`` on issued flops, with the HBM traffic per launch that the rocprofv3
    FETCH_SIZE/WRITE_SIZE passes recorded in profiles/traffic_<workload>.md (null when that
    file is absent), that traffic's rate against the 8 TB/s HBM peak (``hbm_frac``), and
    ``bound`` the resource with the larger fraction;
  * the other BASELINE configs (``gqa``, ``long``: the same per-kernel figures; ``gpt``: the
    GPT training step, tokens/s);
  * the box's sustained MFMA rate (``mfma_ceiling``): a probe kernel issuing only
    fp16 MFMAs on every CU for ~10 ms, its rate and clock (context only);
  * the CPU baseline: the repository's CPU restatement of model.py (oracle,
    fp32) on a time-bounded sample of the same workload;
  * decode steps (``co_alibi_decode``: one query per head against a key/value
    cache) of the decode workloads, against the HBM roofline: algorithmic bytes
    are the cache rows read plus q and o.
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
    # The GPU's clock ramps up over the first ~20 steps of a fresh process (about 0.95 ms per
    # step at first, 0.85 ms from the third 10-step round on, at the headline), so the default
    # warm-up runs 50 untimed steps before the timed ones.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="headline", choices=["headline", "gqa", "long", "cpu", "gpt"],
                    help="attention workload (BASELINE configs[0..3]) or the GPT training step (configs[4])")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="CPU work budget of the CPU-baseline sample in seconds (0 disables it)")
    ap.add_argument("--kernel-reps", type=int, default=10, help="launches per kernel and round in the per-kernel timing")
    ap.add_argument("--kernel-rounds", type=int, default=5, help="rounds of the per-kernel timing (median reported)")
    ap.add_argument("--no-sdpa", dest="sdpa", action="store_false",
                    help="skip the torch SDPA (plain causal attention) comparison")
    ap.add_argument("--no-decode", dest="decode", action="store_false",
                    help="skip the decode-step measurement (co_alibi_decode over a key/value cache)")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="skip the other BASELINE configs (gqa, long, gpt) in the attention run")
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


def cpu_baseline(w, budget_s: float):
    """Times the CPU oracle (fp32 restatement of model.py, fwd + explicit bwd) on the same workload.

    (batch, head) slices are processed in order until ``budget_s`` seconds of CPU work have been
    spent (at least one slice); the rate is algorithmic TFLOP/s of the slices processed.
    """
    import torch

    from co_alibi_attn.profiling import attention_flops
    from co_alibi_attn.workloads import make_inputs
    from oracle import co_alibi_ref as ref

    # Every core of this process's affinity, within the CPU share the host grants one GPU's jobs
    # (OMP_NUM_THREADS, 16 on the MI355X boxes): the share, not the whole host, is this run's CPU.
    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    cores = min(affinity, share) if share > 0 else affinity
    torch.set_num_threads(cores)
    q, k, v, do = (t.float() for t in make_inputs(w, seed=0))
    lam = ref.slopes(w.heads_q, w.bias_max, dtype=w.dtype).float()
    scale = 1.0 / math.sqrt(w.head_dim)
    done, secs = [], 0.0
    for b in range(w.batch):
        for h in range(w.heads_q):
            t0 = time.perf_counter()
            ref.forward(q, k, v, lam, causal=w.causal, scale=scale, heads=[(b, h)])
            ref.backward(do, q, k, v, lam, causal=w.causal, scale=scale, heads=[(b, h)])
            secs += time.perf_counter() - t0
            done.append((b, h))
            if secs >= budget_s:
                break
        if secs >= budget_s:
            break
    fwd, bwd = attention_flops(1, len(done), w.seq, w.seq, w.head_dim, w.causal)
    host_cores = os.cpu_count()
    sample = (f"{w.name} workload, {len(done)} of {w.batch * w.heads_q} (batch, head) slices "
              f"(first: {done[0]}, last: {done[-1]}), fwd+bwd fp32, {secs:.1f} s on {cores} threads "
              f"(CPU share of one GPU: OMP_NUM_THREADS={share or 'unset'}; affinity {affinity} cores, host "
              f"{host_cores}) of {cpu_model_name()}")
    return {"value": round((fwd + bwd) / secs / 1e12, 5), "unit": "TFLOPS", "cores": cores, "kind": "port",
            "sample": sample, "seconds": round(secs, 3), "affinity_cores": affinity, "host_cores": host_cores, "cpu_model": cpu_model_name()}


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


def gpt_measure(steps: int, warmup: int) -> dict:
    """the GPT training step (fwd + bwd + AdamW, bf16 autocast), timed over
    ``steps`` steps after ``warmup``; also Co-ALiBi attention alone at the same shape."""
    import torch

    from co_alibi_attn.gpt import GPT, GPTConfig, make_optimizer, synthetic_batch, train_step

    cfg, batch, seq = GPTConfig(), 8, 1024
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = GPT(cfg).to(dev)
    opt = make_optimizer(model)
    idx, tgt = synthetic_batch(cfg, batch, seq, seed=0, device=dev)
    print(f"[bench] GPT {cfg.n_layer}L d{cfg.d_model} H{cfg.n_head} vocab {cfg.vocab}: "
          f"{model.n_params() / 1e6:.1f}M params, B{batch} S{seq}", file=sys.stderr, flush=True)
    for _ in range(warmup):
        train_step(model, opt, idx, tgt)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        loss = train_step(model, opt, idx, tgt)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # Attention alone at the same shape (fwd + bwd), to state its share of the step.
    from co_alibi_attn import co_alibi_attention

    hd = cfg.d_model // cfg.n_head
    gen = torch.Generator().manual_seed(1)
    q, k, v, do = (torch.randn(batch, cfg.n_head, seq, hd, generator=gen).to(torch.bfloat16).to(dev)
                   for _ in range(4))
    q.requires_grad_(True), k.requires_grad_(True), v.requires_grad_(True)
    for _ in range(3):
        co_alibi_attention(q, k, v).backward(do)
    torch.cuda.synchronize()
    start.record()
    for _ in range(10):
        co_alibi_attention(q, k, v).backward(do)
    end.record()
    torch.cuda.synchronize()
    attn_ms = start.elapsed_time(end) / 10 * cfg.n_layer
    print(f"[bench] GPT step {ms:.3f} ms, {batch * seq / (ms * 1e-3):.0f} tokens/s", file=sys.stderr, flush=True)
    out = {
        "metric": "GPT training step throughput (tokens/s), 12L d768 H12 Co-ALiBi, B8 S1024",
        "value": round(batch * seq / (ms * 1e-3), 1), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 3), "dtype": "bf16",
        "data": "synthetic (uniform-random token ids), random-init weights",
        "config": {"workload": "GPT training step (fwd+bwd+AdamW), BASELINE configs[4]", "layers": cfg.n_layer,
                   "d_model": cfg.d_model, "heads": cfg.n_head, "vocab": cfg.vocab, "global_batch": batch,
                   "seq_len": seq, "params": model.n_params()},
        "final_loss": round(loss.item(), 4),
        "attention_ms_per_step": round(attn_ms, 3),
        "attention_share": round(attn_ms / ms, 3),
    }
    del model, opt
    torch.cuda.empty_cache()
    return out


def gpt_bench(args) -> None:
    """``--workload gpt``: the GPT training step as the line's metric."""
    out = gpt_measure(args.steps, args.warmup)
    out.update({"n_gpus": 1, "higher_is_better": True, "scaling": "weak", "vs_baseline": None})
    print(json.dumps(out), flush=True)


def decode_bench(args):
    """Decode steps (split + merge kernels through the C ABI) of every decode workload: HBM roofline."""
    import torch

    from co_alibi_attn.profiling import DecodeSet
    from co_alibi_attn.workloads import DECODE_WORKLOADS

    out = {}
    for name, w in DECODE_WORKLOADS.items():
        ds = DecodeSet(w)
        ds.step()
        torch.cuda.synchronize()
        ds.time(10)
        ms = sorted(ds.time(max(args.kernel_reps, 20)) for _ in range(args.kernel_rounds))[args.kernel_rounds // 2]
        gbs = ds.bytes / (ms * 1e-3) / 1e9
        out[name] = {"config": {"batch": w.batch, "heads_q": w.heads_q, "heads_kv": w.heads_kv, "seq_kv": w.seq_kv,
                                "head_dim": w.head_dim, "dtype": str(w.dtype).split(".")[-1]},
                     "us_per_step": round(ms * 1e3, 2), "bytes_per_step": ds.bytes,
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gbs / HBM_PEAK_GBS, 4)}}
        print(f"[bench] decode {name}: {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
        del ds
        torch.cuda.empty_cache()
    return out


def time_steps(step, steps: int, warmup: int) -> float:
    """ms per step over ``steps`` calls of ``step`` after ``warmup`` untimed ones (HIP events)."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def kernel_figures(ks, args, peak: float) -> dict:
    """Per-kernel medians of interleaved timing rounds (KernelSet ks, its skip setting), with
    effective (algorithmic) and issued (from the recorded kstart) TFLOP/s."""
    ks.prime()
    import torch

    torch.cuda.synchronize()
    kstart = ks.kstart()
    names = list(ks.kernels) + (["coalibi_fwd_kernel (inference)"] if ks.skip else [])
    timed = {name: [] for name in names}
    for _ in range(args.kernel_rounds):
        for name in names:
            timed[name].append(ks.time(name, args.kernel_reps))
    out = {}
    for name in names:
        ms = sorted(timed[name])[len(timed[name]) // 2]
        charged = ks.charged_flops("coalibi_fwd_kernel" if name.endswith("(inference)") else name)
        issued = ks.issued_flops(name, kstart)
        out[name] = {"ms": round(ms, 4),
                     "effective_tflops": round(charged / (ms * 1e-3) / 1e12, 2),
                     "charged_gflop": round(charged / 1e9, 2),
                     "issued_gflop": None if issued is None else round(issued / 1e9, 2),
                     "issued_tflops": None if issued is None else round(issued / (ms * 1e-3) / 1e12, 2),
                     "mfma_frac": None if issued is None else round(issued / (ms * 1e-3) / 1e12 / peak, 4)}
    return out


def attention_measure(w, args, dev, detail: bool) -> dict:
    """One attention workload: the drop-in step (skip on and off) and the three kernels through the
    C ABI (skip on and off).  ``detail`` adds the inference forward and the processed share."""
    import torch

    from co_alibi_attn import _native, co_alibi_attention
    from co_alibi_attn.profiling import KernelSet, attention_flops

    dtype_name = {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[w.dtype]
    peak = MFMA_PEAK_TFLOPS[dtype_name]
    fwd_flops, bwd_flops = attention_flops(w.batch, w.heads_q, w.seq, w.seq, w.head_dim, w.causal)
    from co_alibi_attn.workloads import make_inputs

    q, k, v, do = make_inputs(w, seed=0, device=dev)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    print(f"[bench] workload {w.name}: B{w.batch} Hq{w.heads_q} Hkv{w.heads_kv} S{w.seq} D{w.head_dim} "
          f"{dtype_name} causal={w.causal}", file=sys.stderr, flush=True)

    def step():
        q.grad = k.grad = v.grad = None
        o = co_alibi_attention(q, k, v, causal=w.causal, bias_max=w.bias_max)
        o.backward(do)

    res = {"config": {"batch": w.batch, "heads_q": w.heads_q, "heads_kv": w.heads_kv, "seq_len": w.seq,
                      "head_dim": w.head_dim, "dtype": dtype_name, "causal": w.causal, "bias_max": w.bias_max}}
    steps, warmup = (args.steps, args.warmup) if detail else (max(args.steps // 4, 10), max(args.warmup // 5, 5))
    res["ms_per_step"] = round(time_steps(step, steps, warmup), 4)
    with _native.tail_skip(False):
        res["ms_per_step_full_work"] = round(time_steps(step, steps, warmup), 4)
    print(f"[bench] {w.name} step {res['ms_per_step']:.3f} ms (tail skip), {res['ms_per_step_full_work']:.3f} ms "
          f"(full work)", file=sys.stderr, flush=True)
    res["effective_tflops"] = round((fwd_flops + bwd_flops) / (res["ms_per_step"] * 1e-3) / 1e12, 2)
    del q, k, v, do

    ks = KernelSet(w, dev)
    ks.skip = True
    on = kernel_figures(ks, args, peak)
    kstart = ks.kstart()
    ks.skip = False
    off = kernel_figures(ks, args, peak)
    fwd_name, p1, p2 = ks.kernels
    res["backward_path"] = ks.path
    res["kernels"] = on
    res["kernels_full_work"] = off

    def fracs(kern):
        fwd_ms = kern[fwd_name]["ms"]
        bwd_ms = kern[p1]["ms"] + kern[p2]["ms"]
        return {"fwd_ms": fwd_ms, "bwd_ms": round(bwd_ms, 4),
                "fwd_tflops": round(fwd_flops / (fwd_ms * 1e-3) / 1e12, 2),
                "bwd_tflops": round(bwd_flops / (bwd_ms * 1e-3) / 1e12, 2),
                "fwd_frac_peak": round(fwd_flops / (fwd_ms * 1e-3) / 1e12 / peak, 4),
                "bwd_frac_peak": round(bwd_flops / (bwd_ms * 1e-3) / 1e12 / peak, 4)}

    res["full_work"] = fracs(off)
    res["tail_skip"] = fracs(on)
    import numpy as np

    from co_alibi_attn.profiling import issued_k16

    full = issued_k16(fwd_name, np.zeros_like(kstart), w.batch, w.heads_q, w.heads_kv, w.seq, w.seq, w.head_dim,
                      w.causal)
    res["tail_skip"]["forward_tiles_processed"] = round(
        issued_k16(fwd_name, kstart, w.batch, w.heads_q, w.heads_kv, w.seq, w.seq, w.head_dim, w.causal) / full, 4)
    print(f"[bench] {w.name} full work: {json.dumps(res['full_work'])}", file=sys.stderr, flush=True)
    print(f"[bench] {w.name} tail skip: {json.dumps(res['tail_skip'])}", file=sys.stderr, flush=True)
    res["_ks"] = ks
    return res


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(each (batch, kv-head) unit runs on one GPU; the op needs no collective)", file=sys.stderr)
        sys.exit(2)

    if args.workload == "gpt":
        gpt_bench(args)
        return

    import torch

    from co_alibi_attn.profiling import attention_flops, read_traffic
    from co_alibi_attn.workloads import WORKLOADS

    w = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    head = attention_measure(w, args, dev, detail=True)
    ks = head.pop("_ks")
    dtype_name = head["config"]["dtype"]
    peak = MFMA_PEAK_TFLOPS[dtype_name]
    fwd_flops, bwd_flops = attention_flops(w.batch, w.heads_q, w.seq, w.seq, w.head_dim, w.causal)
    on, full, skip = head["kernels"], head["full_work"], head["tail_skip"]

    # The roofline of the step's dominant kernel (skip on, as `value` is measured): its issued
    # MFMA work and its HBM traffic, each against its peak; `bound` is the larger fraction.
    names = [n for n in ks.kernels]
    dominant = max(names, key=lambda n: on[n]["ms"])
    traffic = read_traffic(os.path.join(ROOT, "profiles", f"traffic_{w.name}.md")).get(dominant)
    mfma_frac = on[dominant]["mfma_frac"]
    hbm_frac = None if traffic is None else traffic / (on[dominant]["ms"] * 1e-3) / (HBM_PEAK_GBS * 1e9)
    bound = "hbm" if hbm_frac is not None and hbm_frac > mfma_frac else "mfma"
    if bound == "mfma":
        roof = {"bound": "mfma", "achieved": on[dominant]["issued_tflops"], "peak": peak, "unit": "TFLOP/s",
                "frac": mfma_frac}
    else:
        gbs = traffic / (on[dominant]["ms"] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(hbm_frac, 4)}
    roof.update({"kernel": dominant, "traffic": None if traffic is None else round(traffic),
                 "mfma_frac_issued": mfma_frac,
                 "hbm_frac": None if hbm_frac is None else round(hbm_frac, 4),
                 "effective_tflops": on[dominant]["effective_tflops"]})

    from co_alibi_attn.profiling import mfma_probe

    probe_tflops, clock_ghz = mfma_probe(dev)
    print(f"[bench] MFMA probe: {probe_tflops:.0f} TFLOP/s, clock {clock_ghz:.3f} GHz", file=sys.stderr, flush=True)
    del ks
    torch.cuda.empty_cache()

    sdpa_ms, sdpa_mode = None, None
    if args.sdpa:
        sdpa_ms, sdpa_mode = sdpa_measure(w, args, dev)

    ms_step = head["ms_per_step"]
    value = (fwd_flops + bwd_flops) / (ms_step * 1e-3) / 1e12
    out = {
        "metric": "fwd and bwd TFLOPS (and % of MFMA peak) at B4 H16 S4096 D128 fp16 causal",
        "value": round(value, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name,
        "data": "synthetic (seeded N(0,1) inputs of the BASELINE shape)",
        "config": {"workload": f"co_alibi_attention fwd+bwd, {w.name}", "batch": w.batch, "heads_q": w.heads_q,
                   "heads_kv": w.heads_kv, "seq_len": w.seq, "head_dim": w.head_dim, "causal": w.causal,
                   "bias_max": w.bias_max},
        "value_note": "effective TFLOP/s (algorithmic flops over the step time) with the tail skip on; "
                      "fwd_frac_peak / bwd_frac_peak are with the tail skip off (full work)",
        "ms_per_step_full_work": head["ms_per_step_full_work"],
        # the north star's fractions: full work (every visible tile), algorithmic flops / kernel time
        "fwd_ms": full["fwd_ms"],
        "bwd_ms": full["bwd_ms"],
        "fwd_tflops": full["fwd_tflops"],
        "bwd_tflops": full["bwd_tflops"],
        "fwd_frac_peak": full["fwd_frac_peak"],
        "bwd_frac_peak": full["bwd_frac_peak"],
        "tail_skip": skip,
        "fwd_inference_ms": on["coalibi_fwd_kernel (inference)"]["ms"],
        "ref_convention_tflops": {"fwd": round(2 * fwd_flops / (full["fwd_ms"] * 1e-3) / 1e12, 2),
                                  "bwd": round(4 * fwd_flops / (full["bwd_ms"] * 1e-3) / 1e12, 2)},
        "backward_path": head["backward_path"],
        "kernels": on,
        "kernels_full_work": head["kernels_full_work"],
        # The full-work fractions against the probe's measured MFMA-only rate (its clock drops
        # below the published 2.4 GHz under MFMA-only load; the attention kernels, which mix in
        # VALU work, run nearer to it), as context beside the fractions of the published peak.
        "mfma_ceiling": {"probe_fp16_tflops": round(probe_tflops, 1), "clock_ghz": round(clock_ghz, 3),
                         "fwd_frac_of_probe": round(full["fwd_tflops"] / probe_tflops, 4),
                         "bwd_frac_of_probe": round(full["bwd_tflops"] / probe_tflops, 4)},
        "sdpa_ms_per_step": None if sdpa_ms is None else round(sdpa_ms, 4),
        "sdpa_mode": sdpa_mode,
        "coalibi_over_sdpa": None if sdpa_ms is None else round(ms_step / sdpa_ms, 3),
        "roofline": roof,
    }
    if args.configs and w.name == "headline":
        for name in ("gqa", "long"):
            r = attention_measure(WORKLOADS[name], args, dev, detail=False)
            r.pop("_ks")
            torch.cuda.empty_cache()
            out[name] = r
        out["gpt"] = gpt_measure(max(args.steps // 5, 10), max(args.warmup // 5, 5))
    if args.decode:
        out["decode"] = decode_bench(args)
    if args.cpu_seconds > 0:
        print("[bench] CPU baseline ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
        out["cpu_config0_ms"] = round(cpu_config_timing(), 3)
    print(json.dumps(out), flush=True)


def sdpa_measure(w, args, dev):
    """Plain causal attention at the same shape and dtype (torch SDPA on ROCm), fwd + bwd: the cost of
    Co-ALiBi relative to ordinary attention.  Grouped heads go in with enable_gqa; where that path is
    unavailable, K and V are expanded to the query heads outside the timed region."""
    import torch
    import torch.nn.functional as F

    from co_alibi_attn.workloads import make_inputs

    q, k, v, do = make_inputs(w, seed=0, device=dev)
    qs, ks_, vs = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    gqa = w.heads_q != w.heads_kv

    def sdpa_step(kk, vv, **kw):
        qs.grad = ks_.grad = vs.grad = None
        F.scaled_dot_product_attention(qs, kk, vv, is_causal=w.causal, **kw).backward(do)

    run = lambda: sdpa_step(ks_, vs)  # noqa: E731
    mode = "mha"
    if gqa:
        try:
            sdpa_step(ks_, vs, enable_gqa=True)
            run = lambda: sdpa_step(ks_, vs, enable_gqa=True)  # noqa: E731
            mode = "enable_gqa"
        except RuntimeError:
            g = w.heads_q // w.heads_kv
            kx = ks_.detach().repeat_interleave(g, dim=1).requires_grad_(True)
            vx = vs.detach().repeat_interleave(g, dim=1).requires_grad_(True)
            run = lambda: sdpa_step(kx, vx)  # noqa: E731
            mode = "expanded kv"
    ms = time_steps(run, args.steps, 3)
    print(f"[bench] torch SDPA causal fwd+bwd ({mode}): {ms:.3f} ms/step", file=sys.stderr, flush=True)
    return ms, mode


if __name__ == "__main__":
    main()
