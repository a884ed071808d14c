"""Seeded synthetic MoE inputs shared by the tests and the benchmark.

Configurations follow the benchmark definitions: hidden states ~ N(0, 1), router and expert
weights ~ N(0, 0.02), generated on the CPU with torch.Generator and cast to the layer's dtypes.
"""
from dataclasses import dataclass
import math

import torch


@dataclass(frozen=True)
class Case:
    name: str
    T: int
    d: int
    E: int
    k: int
    H: int
    score_fn: int = 0      # 0 softmax, 1 sigmoid
    activation: int = 0    # 0 SwiGLU, 1 ReLU^2
    shared_H: int = 0      # hidden width of the shared expert, 0 = none
    zipf_bias: float = 0.0  # s of the Zipf logit bias, 0 = none
    seed: int = 0


CONFIGS = {
    1: Case("cpu-ref-T512-d256-E8-k2", 512, 256, 8, 2, 512),
    2: Case("bf16-T16384-d1024-E32-k4", 16384, 1024, 32, 4, 512),
    3: Case("bf16-skew-T32768-d2048-E64-k8", 32768, 2048, 64, 8, 1024, zipf_bias=1.2),
    4: Case("bf16-deepseek-T8192-d2048-E128-k8-sigmoid-shared", 8192, 2048, 128, 8, 768,
            score_fn=1, shared_H=1536),
    5: Case("fp8-T64-d4096-E128-k8", 64, 4096, 128, 8, 1536),
    # the registered T3 expert cell moe-T3-L20 (width 1280, 256 experts, top-8, ReLU^2 experts
    # and one shared expert of width 320; configs/scaling/t3.json) on a 8 x 2048-token batch
    6: Case("t3-moe-T3-L20-T16384-d1280-E256-k8-relu2-H320-shared", 16384, 1280, 256, 8, 320,
            activation=1, shared_H=320),
}


def zipf_bias(E, s):
    """2 * log(Zipf(s) weight of rank e+1): rank 1 gets 0, then -2 s log(rank)."""
    return torch.tensor([2.0 * (-s * math.log(r + 1)) for r in range(E)], dtype=torch.float32)


def make_inputs(case, device="cpu"):
    """x bf16 [T, d]; router fp32 [E, d]; w1 fp32 [E, F, d]; w2 fp32 [E, d, H] (+ shared, bias)."""
    g = torch.Generator().manual_seed(case.seed)
    F = 2 * case.H if case.activation == 0 else case.H
    x = torch.randn(case.T, case.d, generator=g).to(torch.bfloat16)
    router = torch.randn(case.E, case.d, generator=g) * 0.02
    w1 = torch.randn(case.E, F, case.d, generator=g) * 0.02
    w2 = torch.randn(case.E, case.d, case.H, generator=g) * 0.02
    out = dict(x=x, router=router, w1=w1, w2=w2, shared_w1=None, shared_w2=None, bias=None)
    if case.shared_H:
        Fs = 2 * case.shared_H if case.activation == 0 else case.shared_H
        out["shared_w1"] = torch.randn(1, Fs, case.d, generator=g) * 0.02
        out["shared_w2"] = torch.randn(1, case.d, case.shared_H, generator=g) * 0.02
    if case.zipf_bias:
        out["bias"] = zipf_bias(case.E, case.zipf_bias)
    if device != "cpu":
        out = {k: (v.to(device) if v is not None else None) for k, v in out.items()}
    return out


def make_router_inputs(case):
    """x bf16 [T, d], router fp32 [E, d] and the logit bias (or None) of make_inputs(case), drawn
    without the expert weights: x and the router come first from the same generator, so the
    values are identical."""
    g = torch.Generator().manual_seed(case.seed)
    x = torch.randn(case.T, case.d, generator=g).to(torch.bfloat16)
    router = torch.randn(case.E, case.d, generator=g) * 0.02
    return x, router, (zipf_bias(case.E, case.zipf_bias) if case.zipf_bias else None)


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()
