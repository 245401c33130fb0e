"""The torch operators co_alibi::fwd / bwd / decode on an MI355X: torch.library.opcheck,
torch.compile with fullgraph=True (no graph break at the native launches) against eager,
and capture of forward + backward + decode in one CUDA (HIP) graph whose replays, with
new inputs and eager work between them, match eager bit for bit."""
import math

import pytest
import torch

from co_alibi_attn import co_alibi_attention
from co_alibi_attn.co_alibi_attn import _get_coalibi_slopes

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def make(B, Hq, Hkv, S, D, dtype, seed=0, skv=None):
    g = torch.Generator().manual_seed(seed)
    skv = S if skv is None else skv
    q = (torch.randn(B, Hq, S, D, generator=g) * 0.5).to(dtype).to(DEV)
    k = (torch.randn(B, Hkv, skv, D, generator=g) * 0.5).to(dtype).to(DEV)
    v = (torch.randn(B, Hkv, skv, D, generator=g) * 0.5).to(dtype).to(DEV)
    do = torch.randn(B, Hq, S, D, generator=g).to(dtype).to(DEV)
    return q, k, v, do


def slopes(hq, dtype):
    return (2.0 * _get_coalibi_slopes(hq)).to(DEV, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["float16", "float32"])
def test_opcheck_fwd_bwd(dtype):
    print(f"opcheck fwd/bwd {dtype}", flush=True)
    q, k, v, do = make(1, 4, 2, 96, 64, dtype)
    sl, scale = slopes(4, dtype), 1 / 8
    grads = tuple(t.clone().requires_grad_() for t in (q, k, v))
    torch.library.opcheck(torch.ops.co_alibi.fwd, (q, k, v, sl, True, scale, False))
    # With the tail skip on, every word of the saved statistics is written (header, kstart, key
    # norms, work orders), so eager and AOT-traced outputs compare in full, causal or not.
    torch.library.opcheck(torch.ops.co_alibi.fwd, (*grads, sl, False, scale, True))
    torch.library.opcheck(torch.ops.co_alibi.fwd, (*grads, sl, True, scale, True))
    o, lse, stats = torch.ops.co_alibi.fwd(q, k, v, sl, True, scale, True)
    torch.library.opcheck(torch.ops.co_alibi.bwd, (do, q, k, v, o, lse, stats, sl, True, scale))
    torch.library.opcheck(torch.ops.co_alibi.bwd_dq, (do, q, k, v, o, lse, stats, sl, True, scale))
    dq_full = torch.ops.co_alibi.bwd(do, q, k, v, o, lse, stats, sl, True, scale)[0]
    assert torch.equal(torch.ops.co_alibi.bwd_dq(do, q, k, v, o, lse, stats, sl, True, scale), dq_full)


def test_opcheck_decode():
    print("opcheck decode", flush=True)
    q, k, v, _ = make(2, 8, 2, 1, 64, torch.bfloat16, skv=600)
    lens = torch.tensor([600, 257], dtype=torch.int32, device=DEV)
    sl = slopes(8, torch.bfloat16)
    torch.library.opcheck(torch.ops.co_alibi.decode, (q, k, v, sl, None, 600, 0.125, True))
    torch.library.opcheck(torch.ops.co_alibi.decode, (q, k, v, sl, lens, 600, 0.125, False))


def test_compile_fullgraph_matches_eager():
    """A loss over co_alibi_attention compiled as one graph (aot_eager: the same kernels, traced
    through the fake implementations and AOT autograd) gives eager's loss and gradients."""
    print("torch.compile fullgraph", flush=True)
    q, k, v, _ = make(2, 8, 2, 200, 64, torch.bfloat16, seed=3)
    w = torch.randn(2, 8, 200, 64, generator=torch.Generator().manual_seed(4)).to(DEV)

    def step(q, k, v):
        return (co_alibi_attention(q, k, v).float() * w).sum()

    def run(fn):
        leaves = [t.clone().requires_grad_() for t in (q, k, v)]
        loss = fn(*leaves)
        loss.backward()
        return loss.detach(), [t.grad for t in leaves]

    loss_e, grads_e = run(step)
    torch._dynamo.reset()
    loss_c, grads_c = run(torch.compile(step, fullgraph=True, backend="aot_eager"))
    torch.cuda.synchronize()
    assert torch.equal(loss_c, loss_e)
    for name, a, b in zip("qkv", grads_c, grads_e):
        assert torch.equal(a, b), f"d{name} differs between compiled and eager"


def test_graph_capture_replays_match_eager():
    """Forward, backward and a decode step captured in one graph.  Each of three replays
    follows new values copied into the static inputs and unrelated eager work, and must equal
    the eager results for those values exactly (the kernels are deterministic)."""
    print("graph capture", flush=True)
    B, Hq, Hkv, S, D, dt = 1, 8, 2, 320, 128, torch.float16
    scale = 1 / math.sqrt(D)
    sl = slopes(Hq, dt)
    q, k, v, do = make(B, Hq, Hkv, S, D, dt, seed=10)
    qd = q[:, :, -1:].clone()

    def work():
        o, lse, stats = torch.ops.co_alibi.fwd(q, k, v, sl, True, scale, True)
        dq, dk, dv = torch.ops.co_alibi.bwd(do, q, k, v, o, lse, stats, sl, True, scale)
        od, lsed = torch.ops.co_alibi.decode(qd, k, v, sl, None, S, scale, True)
        return o, lse, dq, dk, dv, od, lsed

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    torch.cuda.synchronize()

    for rep in range(3):
        nq, nk, nv, ndo = make(B, Hq, Hkv, S, D, dt, seed=100 + rep)
        for dst, src in ((q, nq), (k, nk), (v, nv), (do, ndo), (qd, nq[:, :, -1:])):
            dst.copy_(src)
        torch.cuda.synchronize()
        want = work()  # eager, on the same static inputs
        junk = torch.randn(4096, device=DEV).square().sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for name, got, ref in zip(("o", "lse", "dq", "dk", "dv", "decode o", "decode lse"), outs, want):
            assert torch.equal(got, ref), f"replay {rep}: {name} differs from eager"
        print(f"  replay {rep} matches eager", flush=True)


@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")  # leaves first used on the warm-up stream
def test_public_function_captures_in_a_graph():
    """After one eager call (which puts the slopes on the device), co_alibi_attention and its
    backward through torch.autograd.grad capture into a graph: the public path has no host
    synchronisation.  Replays with new inputs equal eager."""
    print("graph capture of co_alibi_attention", flush=True)
    B, Hq, Hkv, S, D, dt = 2, 8, 4, 200, 64, torch.bfloat16
    q, k, v, do = make(B, Hq, Hkv, S, D, dt, seed=20)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]

    def step():
        o = co_alibi_attention(*leaves)
        return (o, *torch.autograd.grad(o, leaves, do))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for rep in range(2):
        nq, nk, nv, ndo = make(B, Hq, Hkv, S, D, dt, seed=200 + rep)
        with torch.no_grad():
            for dst, src in zip((*leaves, do), (nq, nk, nv, ndo)):
                dst.copy_(src)
        torch.cuda.synchronize()
        want = step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("o", "dq", "dk", "dv"), outs, want):
            assert torch.equal(got, ref), f"replay {rep}: {name} differs from eager"
