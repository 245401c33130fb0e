"""GPT training-step harness: the caller of the attention op.

CPU tests run the model with the oracle's differentiable attention (checker
only); GPU tests run the native kernels through the drop-in API and compare one
step against the same weights on the CPU with the oracle attention.
"""
from __future__ import annotations

import copy
import math

import pytest
import torch

from co_alibi_attn.gpt import GPT, GPTConfig, make_optimizer, synthetic_batch, train_step
from oracle import co_alibi_ref as ref

TINY = GPTConfig(n_layer=2, n_head=2, d_model=128, vocab=97)


def oracle_attention(q, k, v, causal=True, sm_scale=None, bias_max=8.0):
    """Same surface and slope rule as co_alibi_attention, computed by the CPU oracle in fp32."""
    lam = ref.slopes(q.shape[1], bias_max, dtype=q.dtype).float()
    out = ref.forward_autograd(q.float(), k.float(), v.float(), lam, causal=causal, scale=sm_scale)
    return out.to(q.dtype)


def expected_params(cfg: GPTConfig) -> int:
    d, f = cfg.d_model, cfg.mlp_ratio * cfg.d_model
    block = 3 * d * d + d * d + (d * f + f) + (f * d + d) + 4 * d  # qkv, proj, mlp, two LayerNorms
    return cfg.vocab * d + cfg.n_layer * block + 2 * d  # tied embedding / head, final LayerNorm


def test_default_config_is_the_benchmark_model():
    cfg = GPTConfig()
    assert (cfg.n_layer, cfg.n_head, cfg.d_model, cfg.vocab) == (12, 12, 768, 50304)
    assert cfg.d_model // cfg.n_head == 64
    model = GPT(cfg, attention=oracle_attention)
    assert model.n_params() == expected_params(cfg)
    assert not any("pos" in n for n, _ in model.named_parameters())  # positions only through Co-ALiBi


def test_twelve_heads_use_the_odd_power_slope_branch():
    lam = ref.slopes(12, 8.0)
    # n = 8: heads 0..7 are 2 * 2^(-(h+1)), heads 8..11 the odd powers 2 * 2^(-(2t+1)/2)
    want = [2.0 * 2.0 ** -(h + 1) for h in range(8)] + [2.0 * 2.0 ** (-(2 * t + 1) / 2) for t in range(4)]
    torch.testing.assert_close(lam.double(), torch.tensor(want, dtype=torch.float64), rtol=3e-7, atol=0)  # fp32 pow


def test_tiny_model_overfits_a_batch_on_cpu():
    torch.manual_seed(0)
    model = GPT(TINY, attention=oracle_attention)
    opt = make_optimizer(model, lr=3e-3)
    idx, tgt = synthetic_batch(TINY, batch=2, seq=16, seed=1)
    losses = [train_step(model, opt, idx, tgt, autocast_dtype=None).item() for _ in range(25)]
    assert all(math.isfinite(x) for x in losses)
    assert losses[0] == pytest.approx(math.log(TINY.vocab), rel=0.05)  # near-uniform predictions at init
    assert losses[-1] < losses[0] - 1.0


@pytest.mark.gpu
def test_gpt_step_matches_oracle_attention_fp32():
    """One fp32 step: native attention on cuda:0 vs the oracle attention on the CPU, same weights."""
    from co_alibi_attn import co_alibi_attention

    torch.manual_seed(0)
    cpu_model = GPT(TINY, attention=oracle_attention)
    gpu_model = copy.deepcopy(cpu_model)
    for blk in gpu_model.blocks:
        blk.attn.attention = co_alibi_attention
    gpu_model = gpu_model.to("cuda:0")
    idx, tgt = synthetic_batch(TINY, batch=2, seq=64, seed=3)
    _, loss_cpu = cpu_model(idx, tgt)
    loss_cpu.backward()
    _, loss_gpu = gpu_model(idx.cuda(), tgt.cuda())
    loss_gpu.backward()
    assert abs(loss_gpu.item() - loss_cpu.item()) < 1e-4
    for (name, pc), (_, pg) in zip(cpu_model.named_parameters(), gpu_model.named_parameters()):
        scale = pc.grad.abs().max().item() + 1e-12
        err = (pg.grad.cpu() - pc.grad).abs().max().item()
        assert err <= 1e-3 * scale + 1e-6, f"{name}: grad max-abs {err:.3e} (scale {scale:.3e})"


@pytest.mark.gpu
def test_gpt_benchmark_config_trains_in_bf16():
    """BASELINE configs[4] shape (B=8, S=1024, bf16 autocast, AdamW): finite, decreasing loss on a fixed batch."""
    torch.manual_seed(0)
    cfg = GPTConfig()
    model = GPT(cfg).to("cuda:0")
    opt = make_optimizer(model, lr=1e-3)
    idx, tgt = synthetic_batch(cfg, batch=8, seq=1024, seed=0, device="cuda:0")
    losses = [train_step(model, opt, idx, tgt).item() for _ in range(6)]
    print("bf16 GPT losses:", [f"{x:.3f}" for x in losses])
    assert all(math.isfinite(x) for x in losses)
    assert losses[0] == pytest.approx(math.log(cfg.vocab), rel=0.05)
    assert losses[-1] < losses[0] - 0.05
