"""Kernel-level measurement: C-ABI launchers over one workload's buffers, and rocprofv3 summaries.

``bench.py`` times the three kernels with :class:`KernelSet`.  Run on its own,
this file is the program that ``rocprofv3`` wraps for the counter passes, and
it turns rocprofv3's CSV output into the short text summaries kept beside the
benchmark:

  python3 co_alibi_attn/profiling.py run --workload headline --reps 3 [--full-work] [--issued-out F]
      one 1 GiB device-to-device copy (the HBM-counter calibration: it reads
      and writes exactly 1 GiB), then each kernel ``reps`` times, nothing else
      (a decode workload, e.g. ``--workload decode_serving``, runs ``reps``
      decode steps instead: the split and the merge kernel); ``--full-work``
      switches the tail skip off; ``--issued-out`` writes the 32x32x16 products
      each kernel issues per launch, counted from the recorded kstart (JSON)
  python3 co_alibi_attn/profiling.py stats DIR --command CMD --out FILE
      per-kernel duration table from ``rocprofv3 --kernel-trace --stats``
  python3 co_alibi_attn/profiling.py traffic FETCH_DIR WRITE_DIR --command CMD --out FILE
      HBM bytes per launch from a ``--pmc FETCH_SIZE`` and a ``--pmc WRITE_SIZE``
      pass, each scaled by what the same counter reads for the calibration copy
  python3 co_alibi_attn/profiling.py counters DIR_A DIR_B --command CMD --out FILE [--issued F]
      per-kernel shader counters (MFMA and VALU busy, instruction mix, LDS bank
      conflicts) from the two ``--pmc`` passes of COUNTER_PASSES, with the HBM
      rate from the traffic and duration summaries when they are given, and the
      MFMA instructions per launch beside the products counted from kstart

Flop accounting.  The algorithmic work is the FlashAttention convention:
forward 2 products (QK^T, PV) and backward 5 (S, dS, dV, dQ, dK), each
2*B*Hq*D flops per (query, key) pair, halved for causal.  The forward kernel is
charged its 2 products.  On the score-store path backward pass 1 issues S, dS
and dQ and pass 2 (coalibi_bwd_dkdv_store_kernel) dV and dK: each is charged
what it issues.  On the recompute path pass 2 (coalibi_bwd_dkdv_kernel) issues S,
dS, dV and dK and is charged all four, and pass 1 is charged the dQ product only
(its S and dS are counted as issued, not charged).  Either way the charged
backward work is exactly 2.5x the forward's: it is the work the reference's
kernels do (every visible tile), and charged flops over time is the *effective*
rate.  The *issued* flops are what the MFMA units actually execute: with the tail
skip the kernels leave out the keys the forward recorded as negligible (kstart), and
every kernel also issues its masked diagonal tiles whole.  issued_k16 counts them
from the recorded kstart by each kernel's own loop bounds, one 32x32x16 product
(32768 flops, one MFMA instruction in fp16/bf16) per unit; a fraction of the MFMA
peak is taken on issued flops only.
"""
from __future__ import annotations

import argparse
import csv
import glob
import math
import os
import sys
from collections import defaultdict

if __package__ in (None, ""):
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

CALIBRATION_BYTES = 1 << 30
KERNELS = ("coalibi_fwd_kernel", "coalibi_bwd_dq_kernel", "coalibi_bwd_dkdv_kernel")  # recompute path
STORE_KERNELS = ("coalibi_fwd_kernel", "coalibi_bwd_dq_kernel", "coalibi_bwd_dkdv_store_kernel")
DECODE_KERNELS = ("coalibi_decode_split_kernel", "coalibi_decode_merge_kernel")
# co_alibi_fwd launches the key-norm kernel (max |k| per key chunk, for the tail skip) before
# the forward kernel; per-launch timings of "coalibi_fwd_kernel" through the C ABI include it.
NAMED_KERNELS = KERNELS + STORE_KERNELS[2:] + DECODE_KERNELS + ("coalibi_key_norm_kernel",)
# The two --pmc passes of the counter summary: at most 8 SQ and 2 GRBM counters each.
COUNTER_PASSES = (
    ("SQ_INSTS_VALU", "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU", "SQ_WAVES",
     "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE"),
    ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_LDS_BANK_CONFLICT",
     "SQ_ACTIVE_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE"),
)
MI355X_CUS = 256   # 4 SIMDs each
MI355X_XCDS = 8    # GRBM_GUI_ACTIVE is read once per XCD
# (charged, issued) products per launch, in units of one GEMM of 2*B*Hq*D flops per visible pair.
PRODUCTS = {
    "recompute": {"coalibi_fwd_kernel": (2, 2), "coalibi_bwd_dq_kernel": (1, 3), "coalibi_bwd_dkdv_kernel": (4, 4)},
    "store": {"coalibi_fwd_kernel": (2, 2), "coalibi_bwd_dq_kernel": (3, 3), "coalibi_bwd_dkdv_store_kernel": (2, 2)},
}


def score_store_limit() -> int:
    """Largest backward workspace co_alibi::bwd takes for the score store, in bytes: the
    CO_ALIBI_SCORE_STORE_LIMIT_MB environment variable (16384 by default, 0: never), as the
    torch operator reads it."""
    mb = int(os.environ.get("CO_ALIBI_SCORE_STORE_LIMIT_MB", "") or 16384)
    return max(mb, 0) << 20


K16_FLOPS = 2 * 32 * 32 * 16  # one 32x32x16 MFMA product


def issued_k16(kernel, kstart, batch, heads_q, heads_kv, seq_q, seq_kv, head_dim, causal=True):
    """32x32x16 products a kernel issues for one launch, counted from the forward's recorded
    first processed key per (batch * query head, 128-row block) (``kstart``, int array of shape
    (B*Hq, ceil(Sq/128)); all zeros when the tail skip is off), by the kernel's own loop bounds:

    - forward: 128-row blocks of 4 wavefronts x 32 rows, 64-key tiles from the diagonal tile
      down to kstart; a wavefront skips a tile wholly above its rows; per wavefront tile
      2*D/16 (S^T over two 32-key halves) + 4*DP/32 (PV) products, DP = max(D, 32);
    - pass 1: the same rows with 32-key tiles; per wavefront tile 2*D/16 (S^T, dS^T) + 2*DP/32 (dQ);
    - pass 2 (score store): per 32-row x 32-key unit that holds a visible pair of a processed
      64-key block (kstart <= its first key, rows < Sq, keys < Skv), 4*DP/32 (dV, dK);
    - pass 2 (recompute, wavefront pairs): the same units, 2*D/16 + 4*DP/32 (S^T, dS^T, dV, dK).
    Returns None for a kernel it does not model."""
    import numpy as np

    ks = np.asarray(kstart, dtype=np.int64).reshape(batch * heads_q, -1)
    ks = np.where((ks >= 0) & (ks <= seq_kv), ks, 0)  # as the kernels read it
    nqb = (seq_q + 127) // 128
    KS, DT = head_dim // 16, max(head_dim, 32) // 32
    q0 = np.arange(nqb) * 128
    if kernel in ("coalibi_fwd_kernel", "coalibi_bwd_dq_kernel"):
        bn = 64 if kernel == "coalibi_fwd_kernel" else 32
        per_tile = 2 * KS + (4 if bn == 64 else 2) * DT
        last = np.minimum(q0 + 127, seq_kv - 1) if causal else np.full(nqb, seq_kv - 1)
        nkt = last // bn + 1                                  # (nqb,)
        kt0 = np.minimum(ks // bn, nkt[None, :])              # (BH, nqb)
        total = 0
        for w in range(4):
            wrow0 = q0 + 32 * w
            # tiles kt in [kt0, nkt) the wavefront processes; causal: not wholly above its rows
            hi = np.minimum(nkt, (wrow0 + 31) // bn + 1) if causal else nkt  # exclusive bound
            total += np.clip(hi[None, :] - kt0, 0, None).sum()
        return int(total) * per_tile
    if kernel in ("coalibi_bwd_dkdv_store_kernel", "coalibi_bwd_dkdv_kernel"):
        per_unit = 4 * DT + (2 * KS if kernel == "coalibi_bwd_dkdv_kernel" else 0)
        nkb = (seq_kv + 63) // 64
        kw0 = np.arange(nkb)[:, None] * 64 + np.arange(2)[None, :] * 32          # (nkb, 2) key groups
        qs0 = q0[:, None] + np.arange(4)[None, :] * 32                             # (nqb, 4) row halves
        vis = (kw0[None, None, :, :] < seq_kv) & (qs0[:, :, None, None] < seq_q)  # (nqb, 4, nkb, 2)
        if causal:
            vis &= qs0[:, :, None, None] + 31 >= kw0[None, None, :, :]
        per_rb_kb = vis.sum(axis=(1, 3))                                           # (nqb, nkb)
        proc = ks[:, :, None] <= (np.arange(nkb) * 64)[None, None, :]               # (BH, nqb, nkb)
        return int((proc * per_rb_kb[None, :, :]).sum()) * per_unit
    return None


def attention_flops(batch, heads_q, seq_q, seq_kv, head_dim, causal=True):
    """Algorithmic (forward, backward) flops of one attention call in the FlashAttention convention:
    forward 2 products of 2*B*Hq*D flops per (query, key) pair, over Sq*Skv pairs halved when
    causal, and backward 2.5 times the forward.  The reference's harness counts the full square
    with backward 2x (co_alibi_attn/benchmark_flops.py:139-140), 2x / 1.6x these figures."""
    pairs = seq_q * seq_kv / 2.0 if causal else float(seq_q * seq_kv)
    fwd = 4.0 * batch * heads_q * head_dim * pairs
    return fwd, 2.5 * fwd


class KernelSet:
    """Device buffers of one workload and a launcher per kernel, all through the C ABI on one stream.
    ``path``: "store" or "recompute" backward; by default the one co_alibi::bwd takes.
    ``skip``: the library's tail-skip setting during this set's launches (timing and priming
    switch it for their duration; the backward kernels follow what the forward recorded)."""

    def __init__(self, w, device="cuda:0", seed: int = 0, path: str | None = None, skip: bool = True):
        import torch

        from co_alibi_attn import _native
        from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes
        from co_alibi_attn.workloads import make_inputs

        self.w = w
        self.skip = bool(skip)
        dev = torch.device(device)
        lib = _native.lib()
        B, Hq, Hkv, S, D = w.batch, w.heads_q, w.heads_kv, w.seq, w.head_dim
        self.q, self.k, self.v, self.do = make_inputs(w, seed=seed, device=dev)
        self.lam = (2.0 * _get_coalibi_slopes(Hq, w.bias_max)).to(w.dtype).float().to(dev)
        self.o = torch.empty_like(self.q)
        self.lse = torch.empty(B, Hq, S, device=dev, dtype=torch.float32)
        self.stats = torch.empty(lib.co_alibi_stats_numel(B, Hq, S, S), device=dev, dtype=torch.float32)
        code = _native.DTYPE_CODES[w.dtype]
        store_bytes = lib.co_alibi_bwd_score_store_workspace_bytes(code, B, Hq, Hkv, S, S, D, int(w.causal))
        if path is None:
            path = "store" if 0 < store_bytes <= score_store_limit() else "recompute"
        if path == "store" and store_bytes == 0:
            raise ValueError(f"{w.name}: no score-store path for this dtype / head dim")
        self.path = path
        self.kernels = STORE_KERNELS if path == "store" else KERNELS
        self.ws_bytes = store_bytes if path == "store" else lib.co_alibi_bwd_workspace_bytes(B, Hq, S, S)
        self.ws = torch.empty(self.ws_bytes, device=dev, dtype=torch.uint8)
        self.dq, self.dk, self.dv = (torch.empty_like(t) for t in (self.q, self.k, self.v))
        self.stream = torch.cuda.current_stream(dev)
        shape = (B, Hq, Hkv, S, S, D, int(w.causal), 1.0 / math.sqrt(D), self.stream.cuda_stream)
        p = lambda t: t.data_ptr()  # noqa: E731

        def fwd():
            _native.check(lib.co_alibi_fwd(code, p(self.q), p(self.k), p(self.v), p(self.lam), p(self.o),
                                           p(self.lse), p(self.stats), *shape))

        def dq():
            _native.check(lib.co_alibi_bwd_dq(code, p(self.do), p(self.q), p(self.k), p(self.v), p(self.o),
                                              p(self.lse), p(self.stats), p(self.lam), p(self.dq), p(self.ws),
                                              self.ws_bytes, *shape))

        def dkdv():
            _native.check(lib.co_alibi_bwd_dkdv(code, p(self.do), p(self.q), p(self.k), p(self.v), p(self.lse),
                                                p(self.stats), p(self.lam), p(self.dk), p(self.dv), p(self.ws),
                                                self.ws_bytes, *shape))

        self.ws_inf_bytes = lib.co_alibi_fwd_inference_workspace_bytes(B, Hq, S, S)
        self.ws_inf = torch.empty(self.ws_inf_bytes, device=dev, dtype=torch.uint8)

        def fwd_inference():  # no LSE / stats: the forward of a caller that needs no backward (tail skip included)
            _native.check(lib.co_alibi_fwd_inference(code, p(self.q), p(self.k), p(self.v), p(self.lam), p(self.o),
                                                     p(self.ws_inf), self.ws_inf_bytes, *shape))

        self.launch = dict(zip(self.kernels, (fwd, dq, dkdv)))
        self.launch["coalibi_fwd_kernel (inference)"] = fwd_inference
        self.gemm_flops = attention_flops(B, Hq, S, S, D, w.causal)[0] / 2.0  # one product

    def charged_flops(self, name: str) -> float:
        """Algorithmic (FlashAttention-convention) flops charged to a kernel: the work of every
        visible tile, whatever the tail skip leaves out."""
        return PRODUCTS[self.path][name][0] * self.gemm_flops

    def kstart(self):
        """The forward's recorded first processed key per (batch * query head, 128-row block), as
        a CPU int32 array (after a forward launch of this set)."""
        import torch

        w = self.w
        n = w.batch * w.heads_q * ((w.seq + 127) // 128)
        return self.stats[4:4 + n].view(torch.int32).view(w.batch * w.heads_q, -1).cpu().numpy()

    def issued_flops(self, name: str, kstart=None) -> float | None:
        """Flops the MFMA units execute in one launch of a kernel, from the recorded kstart."""
        w = self.w
        if name == "coalibi_fwd_kernel (inference)":
            name = "coalibi_fwd_kernel"
        n = issued_k16(name, self.kstart() if kstart is None else kstart, w.batch, w.heads_q, w.heads_kv, w.seq,
                       w.seq, w.head_dim, w.causal)
        return None if n is None else n * K16_FLOPS

    def prime(self) -> None:
        """One launch of each kernel in pipeline order, so every input of every kernel is defined."""
        from co_alibi_attn import _native

        with _native.tail_skip(self.skip):
            for name in self.kernels:
                self.launch[name]()

    def time(self, name: str, reps: int) -> float:
        """Average launch duration in ms over ``reps`` back-to-back launches, HIP events on the launch stream."""
        import torch

        from co_alibi_attn import _native

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with _native.tail_skip(self.skip):
            e0.record(self.stream)
            for _ in range(reps):
                self.launch[name]()
            e1.record(self.stream)
            e1.synchronize()
        return e0.elapsed_time(e1) / reps


class DecodeSet:
    """Device buffers of one decode workload and its C-ABI launcher (split + merge kernels)."""

    KERNELS = DECODE_KERNELS

    def __init__(self, w, device="cuda:0", seed: int = 0):
        import torch

        from co_alibi_attn import _native
        from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes
        from co_alibi_attn.workloads import make_decode_inputs

        self.w = w
        dev = torch.device(device)
        lib = _native.lib()
        B, Hq, Hkv, L, D = w.batch, w.heads_q, w.heads_kv, w.seq_kv, w.head_dim
        self.q, self.k, self.v = make_decode_inputs(w, seed=seed, device=dev)
        self.lam = (2.0 * _get_coalibi_slopes(Hq, w.bias_max)).to(w.dtype).float().to(dev)
        self.o = torch.empty_like(self.q)
        self.lse = torch.empty(B, Hq, device=dev, dtype=torch.float32)
        self.ws_bytes = lib.co_alibi_decode_workspace_bytes(B, Hq, L, D)
        self.ws = torch.empty(self.ws_bytes, device=dev, dtype=torch.uint8)
        self.stream = torch.cuda.current_stream(dev)
        code = _native.DTYPE_CODES[w.dtype]
        p = lambda t: t.data_ptr()  # noqa: E731
        args = (code, p(self.q), p(self.k), p(self.v), p(self.lam), 0, p(self.o), p(self.lse), p(self.ws),
                self.ws_bytes, B, Hq, Hkv, L, L, D, 1.0 / math.sqrt(D), self.stream.cuda_stream)

        def step():
            _native.check(lib.co_alibi_decode(*args))

        self.step = step
        elem = self.q.element_size()
        # Algorithmic HBM bytes of one step: the cache rows, q and o.
        self.bytes = w.cache_bytes() + 2 * B * Hq * D * elem

    def time(self, reps: int) -> float:
        """Average step duration in ms over ``reps`` back-to-back steps, HIP events on the launch stream."""
        import torch

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        for _ in range(reps):
            self.step()
        e1.record(self.stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps


def mfma_probe(device="cuda:0", iters: int = 20000, per_cu: int = 2):
    """Sustained MFMA rate and shader clock under MFMA load on every CU.

    Returns (tflops, clock_ghz): fp16 MFMA TFLOP/s from the probe's wall time (HIP events),
    and the clock from the shader-clock / 100 MHz real-time counter ratio of its loops.
    """
    import torch

    from co_alibi_attn import _native

    lib = _native.lib()
    dev = torch.device(device)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks = cus * per_cu
    ticks = torch.zeros(2 * blocks, dtype=torch.int64, device=dev)
    sink = torch.empty(256 * blocks, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    run = lambda: _native.check(lib.co_alibi_probe_mfma(ticks.data_ptr(), sink.data_ptr(), blocks, iters,  # noqa: E731
                                                         stream.cuda_stream))
    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    run()
    e1.record(stream)
    e1.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3
    flops = blocks * 4 * iters * 4 * 2.0 * 32 * 32 * 16  # waves x rounds x MFMAs x flops
    t = ticks.view(blocks, 2).double().cpu()
    clock_ghz = float((t[:, 0] / t[:, 1]).median()) * 0.1  # shader ticks per 10 ns tick
    return flops / sec / 1e12, clock_ghz


def calibration_copy(device="cuda:0", nbytes: int = CALIBRATION_BYTES) -> None:
    """A device-to-device copy of ``nbytes``: it reads and writes exactly ``nbytes`` of HBM."""
    import torch

    a = torch.ones(nbytes // 2, dtype=torch.float16, device=device)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()


def cmd_run(args) -> None:
    import torch

    from co_alibi_attn.workloads import DECODE_WORKLOADS, WORKLOADS

    calibration_copy()
    if args.workload in DECODE_WORKLOADS:
        ds = DecodeSet(DECODE_WORKLOADS[args.workload])
        for _ in range(args.reps):
            ds.step()
        torch.cuda.synchronize()
        print(f"profiling run: {args.workload}, {args.reps} decode steps ({', '.join(DECODE_KERNELS)})", flush=True)
        return
    ks = KernelSet(WORKLOADS[args.workload], skip=not args.full_work)
    for _ in range(args.reps):
        ks.prime()
    torch.cuda.synchronize()
    mode = "full work (tail skip off)" if args.full_work else "tail skip on"
    print(f"profiling run: {args.workload}, {mode}, {args.reps} launches of each of {', '.join(ks.kernels)}",
          flush=True)
    if args.issued_out:
        import json

        w = ks.w
        kstart = ks.kstart()
        issued = {name: issued_k16(name, kstart, w.batch, w.heads_q, w.heads_kv, w.seq, w.seq, w.head_dim, w.causal)
                  for name in ks.kernels}
        with open(args.issued_out, "w") as fh:
            json.dump({"workload": w.name, "mode": mode, "k16_per_launch": issued}, fh)
        print(f"issued 32x32x16 products per launch: {issued}", flush=True)


def _csv_rows(directory: str, suffix: str):
    files = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {directory}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _short(name: str) -> str:
    for k in NAMED_KERNELS:
        if k in name:
            return k
    return name if len(name) <= 60 else name[:57] + "..."


FULL_WORK = " (full work)"


def _mode_split(trace_rows):
    """Per-dispatch rows of a kernel trace, in time order, with each attention kernel named by the
    tail-skip mode it ran in: the forward's template says it (its last argument, the skip), and
    the backward kernels take the mode of the latest forward before them.  Returns
    {name: [duration ns, ...]}."""
    import re

    out = defaultdict(list)
    full = False
    for r in sorted(trace_rows, key=lambda r: int(r["Start_Timestamp"])):
        name = r["Kernel_Name"]
        short = _short(name)
        if short == "coalibi_fwd_kernel":  # the last template argument, demangled or mangled
            m = re.search(r"coalibi_fwd_kernel<[^>]*?,\s*(true|false)\s*>", name) or \
                re.search(r"coalibi_fwd_kernelI.*Lb([01])E", name)
            full = m is not None and m.group(1) in ("false", "0")
        if short in ("coalibi_fwd_kernel", "coalibi_bwd_dq_kernel", "coalibi_bwd_dkdv_kernel",
                     "coalibi_bwd_dkdv_store_kernel") and full:
            short += FULL_WORK
        out[short].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return out


def cmd_stats(args) -> None:
    lines = [f"# rocprofv3 kernel statistics: {args.title}", "", "Command (R is the repository root on the GPU box):", "",
             "```", args.command, "```", "",
             "The summary is written by `python3 co_alibi_attn/profiling.py stats <rocprofv3 output dir>`.", ""]
    traces = glob.glob(os.path.join(args.dir, "**", "*kernel_trace.csv"), recursive=True)
    if traces:
        rows = _csv_rows(args.dir, "kernel_trace.csv")
        per = _mode_split(rows)
        total = sum(sum(v) for v in per.values()) or 1
        lines += ["Per-dispatch durations from the kernel trace.  The forward's template names its tail-skip "
                  f"mode; the backward kernels that follow a forward without the skip are listed as "
                  f"`...{FULL_WORK}`.", "",
                  "| kernel | calls | average (us) | min (us) | max (us) | share of GPU time |",
                  "|---|---:|---:|---:|---:|---:|"]
        for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"| `{k}` | {len(v)} | {sum(v) / len(v) / 1e3:.1f} | {min(v) / 1e3:.1f} | {max(v) / 1e3:.1f} | "
                         f"{100.0 * sum(v) / total:.1f} % |")
    else:
        rows = _csv_rows(args.dir, "kernel_stats.csv")
        lines += ["| kernel | calls | average (us) | min (us) | max (us) | share of GPU time |",
                  "|---|---:|---:|---:|---:|---:|"]
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
            lines.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} % |")
    _write(args.out, lines)


def _per_dispatch(directory: str, counter: str):
    """{kernel name: [counter value per dispatch]} (values of one dispatch summed over their instances)."""
    acc = defaultdict(float)
    names = {}
    for r in _csv_rows(directory, "counter_collection.csv"):
        if r["Counter_Name"] != counter:
            continue
        key = (r["Process_Id"], r["Dispatch_Id"])
        acc[key] += float(r["Counter_Value"])
        names[key] = r["Kernel_Name"]
    out = defaultdict(list)
    for key, val in acc.items():
        out[names[key]].append(val)
    return out


def cmd_traffic(args) -> None:
    lines = [f"# HBM traffic per launch: {args.title}", "", "Commands (R is the repository root on the GPU box):", "",
             "```", args.command, "```", "",
             f"Each counter is read in KiB per dispatch and scaled by the factor that makes the calibration copy "
             f"(a {CALIBRATION_BYTES >> 20} MiB device-to-device copy, `__amd_rocclr_copyBuffer`, the copy "
             f"dispatch with the largest reading) read exactly {CALIBRATION_BYTES >> 20} MiB. The summary is written "
             f"by `python3 co_alibi_attn/profiling.py traffic <fetch dir> <write dir>`.", ""]
    result = {}
    for counter, directory in (("FETCH_SIZE", args.fetch_dir), ("WRITE_SIZE", args.write_dir)):
        per = _per_dispatch(directory, counter)
        copies = [v for n, vals in per.items() if "copyBuffer" in n for v in vals]
        if not copies:
            raise SystemExit(f"no calibration copy dispatch in {directory}")
        cal_kib = max(copies)
        factor = CALIBRATION_BYTES / (cal_kib * 1024.0)
        lines.append(f"- `{counter}`: calibration copy read {cal_kib:.0f} KiB, factor {factor:.4f}")
        for name, vals in per.items():
            k = _short(name)
            if k in NAMED_KERNELS:
                result.setdefault(k, {})[counter] = sum(vals) / len(vals) * 1024.0 * factor
    lines += ["", "| kernel | fetched (MB) | written (MB) | HBM traffic (MB) |", "|---|---:|---:|---:|"]
    for k in NAMED_KERNELS:
        if k in result:
            f, wr = result[k].get("FETCH_SIZE", 0.0), result[k].get("WRITE_SIZE", 0.0)
            lines.append(f"| `{k}` | {f / 1e6:.1f} | {wr / 1e6:.1f} | {(f + wr) / 1e6:.1f} |")
    lines += ["", "Machine-readable (bytes per launch, read by bench.py):", ""]
    for k in NAMED_KERNELS:
        if k in result:
            total = result[k].get("FETCH_SIZE", 0.0) + result[k].get("WRITE_SIZE", 0.0)
            lines.append(f"    traffic_bytes_per_launch {k} {total:.0f}")
    _write(args.out, lines)


def _counters_per_dispatch(directory: str):
    """{kernel: {counter: mean over dispatches of the value summed over its instances}}."""
    acc = defaultdict(float)
    names = {}
    for r in _csv_rows(directory, "counter_collection.csv"):
        key = (r["Process_Id"], r["Dispatch_Id"], r["Counter_Name"])
        acc[key] += float(r["Counter_Value"])
        names[key[:2]] = r["Kernel_Name"]
    per = defaultdict(lambda: defaultdict(list))
    for (pid, did, counter), val in acc.items():
        per[_short(names[(pid, did)])][counter].append(val)
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in per.items()}


def _stats_average_us(path: str):
    """{kernel: average duration in us} from a summary written by ``stats``."""
    out = {}
    if path and os.path.exists(path):
        with open(path) as fh:
            for line in fh:
                cells = [c.strip() for c in line.split("|")]
                if len(cells) > 4 and cells[1].startswith("`"):
                    out[cells[1].strip("`")] = float(cells[3])
    return out


def cmd_counters(args) -> None:
    """Shader counters per kernel.  Normalisation (MI355X: 256 CUs, 1024 SIMDs, 8 XCDs):
    - active cycles per dispatch T = GRBM_GUI_ACTIVE / 8 (the counter is summed over the XCDs);
    - MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 T) (summed over SIMDs);
    - VALU busy = 4 SQ_ACTIVE_INST_VALU / (1024 T) (quad-cycles summed over waves; one VALU
      instruction issues per SIMD and cycle, so this is the SIMDs' VALU-issue share);
    - LDS bank conflicts: SQ_LDS_BANK_CONFLICT cycles per LDS instruction and as a share of
      the cycles the LDS instructions were active (4 SQ_ACTIVE_INST_LDS);
    - HBM rate = traffic bytes per launch / average duration, from the traffic and stats
      summaries."""
    merged = defaultdict(dict)
    for d in args.dirs:
        for k, cs in _counters_per_dispatch(d).items():
            for c, v in cs.items():
                merged[k].setdefault(c, []).append(v)
    data = {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in merged.items()}
    traffic = read_traffic(args.traffic) if args.traffic else {}
    durations = _stats_average_us(args.stats)
    issued = {}
    if args.issued:
        import json

        with open(args.issued) as fh:
            issued = json.load(fh)["k16_per_launch"]
    simds = 4 * MI355X_CUS
    lines = [f"# Shader counters per launch: {args.title}", "", "Commands (R is the repository root on the GPU box):",
             "", "```", args.command, "```", "",
             "The summary is written by `python3 co_alibi_attn/profiling.py counters <pass dirs>`. Definitions "
             "(MI355X: 256 CUs = 1024 SIMDs, 8 XCDs; T = GRBM_GUI_ACTIVE / 8, the active cycles of a dispatch):",
             "",
             "- MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 T);",
             "- VALU busy = 4 SQ_ACTIVE_INST_VALU / (1024 T), the SIMDs' VALU-issue share;",
             "- instruction mix = SQ_INSTS_* per SQ_INSTS_MFMA;",
             "- LDS conflict = SQ_LDS_BANK_CONFLICT cycles per SQ_INSTS_LDS, and as a share of 4 SQ_ACTIVE_INST_LDS;",
             "- HBM GB/s = traffic per launch (`profiles/traffic_*.md`) / average duration "
             "(`profiles/kernel_stats_*.md`" + (", its full-work rows" if args.full_work else "") + ").", "",
             "| kernel | MFMA busy | VALU busy | VALU / MFMA | trans / MFMA | LDS / MFMA | LDS conflict cycles / LDS instr "
             "| conflict share of LDS cycles | HBM GB/s |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for k in NAMED_KERNELS:
        if k not in data:
            continue
        c = data[k]
        t = c.get("GRBM_GUI_ACTIVE", 0.0) / MI355X_XCDS
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        def frac(x):
            return f"{100.0 * x:.1f} %"
        mfma_busy = frac(c["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * t)) if t and "SQ_VALU_MFMA_BUSY_CYCLES" in c else "-"
        valu_busy = frac(4 * c["SQ_ACTIVE_INST_VALU"] / (simds * t)) if t and "SQ_ACTIVE_INST_VALU" in c else "-"
        def per_mfma(name):
            return f"{c[name] / mf:.2f}" if mf and name in c else "-"
        lds = c.get("SQ_INSTS_LDS", 0.0)
        conf = c.get("SQ_LDS_BANK_CONFLICT")
        conf_per = f"{conf / lds:.3f}" if conf is not None and lds else "-"
        lds_cyc = 4 * c.get("SQ_ACTIVE_INST_LDS", 0.0)
        conf_share = frac(conf / lds_cyc) if conf is not None and lds_cyc else "-"
        dk = k + FULL_WORK if args.full_work and k + FULL_WORK in durations else k
        hbm = (f"{traffic[k] / (durations[dk] * 1e-6) / 1e9:.0f}" if k in traffic and durations.get(dk) else "-")
        lines.append(f"| `{k}` | {mfma_busy} | {valu_busy} | {per_mfma('SQ_INSTS_VALU')} | "
                     f"{per_mfma('SQ_INSTS_VALU_TRANS_F32')} | {per_mfma('SQ_INSTS_LDS')} | {conf_per} | {conf_share} | {hbm} |")
    if issued:
        lines += ["", "MFMA instructions per launch (`SQ_INSTS_MFMA`, one per 32x32x16 product in fp16 / bf16) "
                  "against the products each kernel issues by its loop bounds, counted from the recorded first "
                  "processed keys (`profiling.issued_k16`, the `issued_gflop` of bench.py / 32768 flops):", "",
                  "| kernel | SQ_INSTS_MFMA | issued_k16 | ratio | issued GFLOP |", "|---|---:|---:|---:|---:|"]
        for k in NAMED_KERNELS:
            if k in data and k in issued and issued[k]:
                mf = data[k].get("SQ_INSTS_MFMA", 0.0)
                lines.append(f"| `{k}` | {mf:.0f} | {issued[k]} | {mf / issued[k]:.4f} | "
                             f"{issued[k] * K16_FLOPS / 1e9:.2f} |")
    lines += ["", "Raw means per dispatch:", ""]
    for k in NAMED_KERNELS:
        if k in data:
            lines.append(f"- `{k}`: " + ", ".join(f"{c} {v:.4g}" for c, v in sorted(data[k].items())))
    _write(args.out, lines)


def read_traffic(path: str):
    """{kernel: HBM bytes per launch} from a summary written by ``traffic`` (empty if the file is absent)."""
    out = {}
    if not os.path.exists(path):
        return out
    with open(path) as fh:
        for line in fh:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch":
                out[parts[1]] = float(parts[2])
    return out


def _write(path: str, lines) -> None:
    text = "\n".join(lines) + "\n"
    if path == "-":
        sys.stdout.write(text)
        return
    with open(path, "w") as fh:
        fh.write(text)
    print(f"wrote {path}")


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--workload", default="headline")
    r.add_argument("--reps", type=int, default=3)
    r.add_argument("--full-work", action="store_true", help="switch the tail skip off (every key processed)")
    r.add_argument("--issued-out", default=None, help="write the products issued per launch (JSON)")
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--command", required=True)
    s.add_argument("--title", default="headline benchmark")
    s.add_argument("--out", default="-")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--command", required=True)
    t.add_argument("--title", default="headline workload")
    t.add_argument("--out", default="-")
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--command", required=True)
    c.add_argument("--title", default="headline workload")
    c.add_argument("--traffic", default=None, help="summary written by traffic (for the HBM rate)")
    c.add_argument("--stats", default=None, help="summary written by stats (average durations)")
    c.add_argument("--issued", default=None, help="products per launch written by run --issued-out")
    c.add_argument("--full-work", action="store_true",
                   help="the passes ran with the tail skip off: take the stats summary's full-work rows")
    c.add_argument("--out", default="-")
    args = ap.parse_args(argv)
    {"run": cmd_run, "stats": cmd_stats, "traffic": cmd_traffic, "counters": cmd_counters}[args.cmd](args)


if __name__ == "__main__":
    main()
