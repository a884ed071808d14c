"""TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference MoE layer forward.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

What it restates (paths relative to the NextTransformer tree):
  * router logits in fp32: `F.linear(x.float(), W.float())`
    (nexttransformer/scaling/megatron_moe.py:95-99, reference_blocks.py:37). Two flavours:
    `router_logits_reference` is that expression verbatim (torch's BLAS order);
    `router_logits_fixed` is the C restatement with the fixed, documented order that the HIP
    router also follows (oracle/router_ref.c), which makes routing comparable bit for bit.
  * top-k on logits, softmax over the selected (megatron_moe.py:43, reference_blocks.py:37-38);
    sigmoid scores normalised over the selected for the DeepSeek-style config (not in the
    reference; closed form). Ties: the lower expert index ranks first.
  * expert-major, token-ascending permutation, counts (megatron_moe.py:142-144).
  * per-expert FFN: SwiGLU `fc2(silu(g) * u)` with g = fc1 rows [0, H) (MCore
    gated_linear_unit order) or ReLU^2 `fc2(relu(fc1 x)^2)` (megatron_moe.py:23-24,
    lm.py:29-35), applied in an eager per-expert loop as RoutedFFN does
    (reference_blocks.py:39-44), weighted after fc2, accumulated with index_add in ascending
    expert order, plus an optional shared expert (megatron_moe.py:150).
  * auxiliary losses, MCore "aux_loss" type with coefficients from MoERecipe
    (megatron_moe.py:44-45, moe_recipe.py:40-41), in their published closed forms:
    lb = coeff * E / (k T^2) * sum_e (sum_t s_te) * count_e with s = full softmax (or
    sigmoid normalised over all experts); z = coeff * mean_t logsumexp(logits_t)^2.
    Parity against MCore 0.21.0 itself is unpinned (MCore is not installed); these closed
    forms are pinned by invariants in tests/test_oracle_pins.py.
  * fp8: OCP e4m3fn quantisation (per-token activations, 128x128-block weights) and the
    fp32 dequantised reference the fp8 path is scored against.
"""
import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch
from torch.nn import functional as F

_LIB = None
SOFTMAX, SIGMOID = 0, 1
SWIGLU, RELU2 = 0, 1
E4M3_MAX = 448.0


def lib():
    """The compiled C restatement (oracle/_build/liboracle_moe.so); built by oracle.build."""
    global _LIB
    if _LIB is None:
        path = Path(__file__).resolve().parent / "_build" / "liboracle_moe.so"
        if not path.exists():
            from oracle.build import build
            build()
        so = ctypes.CDLL(str(path))
        p = ctypes.c_void_p
        i64, i32 = ctypes.c_int64, ctypes.c_int32
        so.oracle_router_logits.argtypes = [p, i64, p, p, i64, i32, i32, p]
        so.oracle_topk.argtypes = [p, i64, i32, i32, i32, p, p]
        so.oracle_route_plan.argtypes = [p, i64, i32, i32, p, p, p, p]
        for f in (so.oracle_router_logits, so.oracle_topk, so.oracle_route_plan):
            f.restype = None
        _LIB = so
    return _LIB


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def router_logits_fixed(x, w_router, bias=None):
    """fp32 logits [T, E] in the fixed order (see oracle/router_ref.c). x: bf16 [T, d]."""
    x = x.detach().to("cpu", torch.bfloat16).contiguous()
    w = w_router.detach().to("cpu", torch.float32).contiguous()
    T, d = x.shape
    E = w.shape[0]
    out = torch.empty(T, E, dtype=torch.float32)
    b = None if bias is None else bias.detach().to("cpu", torch.float32).contiguous()
    lib().oracle_router_logits(_ptr(x), d, _ptr(w), None if b is None else _ptr(b), T, d, E, _ptr(out))
    return out


def router_logits_reference(x, w_router, bias=None):
    """The reference expression F.linear(x.float(), W.float()) (megatron_moe.py:99)."""
    logits = F.linear(x.detach().cpu().float(), w_router.detach().cpu().float())
    return logits if bias is None else logits + bias.detach().cpu().float()


def topk(logits, k, score_fn=SOFTMAX):
    """(ids int32 [T, k], weights fp32 [T, k]) with the tie rule; descending logit order."""
    logits = logits.detach().to("cpu", torch.float32).contiguous()
    T, E = logits.shape
    ids = torch.empty(T, k, dtype=torch.int32)
    w = torch.empty(T, k, dtype=torch.float32)
    lib().oracle_topk(_ptr(logits), T, E, k, score_fn, _ptr(ids), _ptr(w))
    return ids, w


def route_plan(ids, E):
    """counts [E], offsets [E+1], src_row [T*k], dest [T, k] -- the order of mapping.T.nonzero()."""
    ids = ids.detach().to("cpu", torch.int32).contiguous()
    T, k = ids.shape
    counts = torch.empty(E, dtype=torch.int32)
    offsets = torch.empty(E + 1, dtype=torch.int32)
    src = torch.empty(T * k, dtype=torch.int32)
    dest = torch.empty(T, k, dtype=torch.int32)
    lib().oracle_route_plan(_ptr(ids), T, k, E, _ptr(counts), _ptr(offsets), _ptr(src), _ptr(dest))
    return counts, offsets, src, dest


def full_scores(logits, score_fn=SOFTMAX):
    """Scores over all experts used by the load-balance loss."""
    logits = logits.double()
    if score_fn == SOFTMAX:
        return logits.softmax(-1)
    s = torch.sigmoid(logits)
    return s / s.sum(-1, keepdim=True)


def aux_losses(logits, counts, k, aux_coeff, z_coeff, score_fn=SOFTMAX):
    """(lb, z) in float64: MCore switch load-balance loss and router z-loss, closed forms."""
    T, E = logits.shape
    s = full_scores(logits, score_fn)
    lb = aux_coeff * E / (k * T * T) * (s.sum(0) * counts.double()).sum()
    z = z_coeff * torch.logsumexp(logits.double(), -1).square().mean()
    return lb.item(), z.item()


def act(fc1_out, activation, H):
    if activation == SWIGLU:
        return F.silu(fc1_out[..., :H]) * fc1_out[..., H:]
    return F.relu(fc1_out).square()


def expert_ffn(rows, w1, w2, activation):
    """One expert in fp32 (or the dtype of rows): fc2(act(fc1(rows)))."""
    H = w2.shape[1]
    return act(rows @ w1.t(), activation, H) @ w2.t()


@dataclass
class Weights:
    """Expert weights as the oracle consumes them (any float dtype; used in fp32)."""
    router: torch.Tensor            # [E, d] fp32
    w1: torch.Tensor                # [E, F, d]
    w2: torch.Tensor                # [E, d, H]
    shared_w1: torch.Tensor = None  # [Fs, d]
    shared_w2: torch.Tensor = None  # [d, Hs]
    bias: torch.Tensor = None       # [E] logit bias


def moe_forward(x, weights, k, *, score_fn=SOFTMAX, activation=SWIGLU, aux_coeff=0.01,
                z_coeff=0.001, router="fixed", logits=None, dtype=torch.float32):
    """Full MoE layer forward on the CPU.

    x [T, d] (any float dtype; bf16 inputs are used exactly). Experts run in `dtype`
    (fp32 by default) in an eager per-expert loop with index_add in ascending expert
    order (reference_blocks.py:39-44). Returns a dict with out [T, d] in `dtype`, aux, the
    routing tensors and the plan.
    """
    x = x.detach().cpu()
    if logits is None:
        logits = (router_logits_fixed(x, weights.router, weights.bias) if router == "fixed"
                  else router_logits_reference(x, weights.router, weights.bias))
    E = weights.router.shape[0]
    ids, topw = topk(logits, k, score_fn)
    counts, offsets, src, dest = route_plan(ids, E)
    rows = x.to(dtype)
    out = torch.zeros_like(rows)
    ids64 = ids.long()
    for e in range(E):
        token, slot = torch.where(ids64 == e)
        if token.numel():
            y = expert_ffn(rows[token], weights.w1[e].to(dtype), weights.w2[e].to(dtype), activation)
            out.index_add_(0, token, y * topw[token, slot, None].to(dtype))
    if weights.shared_w1 is not None:
        out = out + expert_ffn(rows, weights.shared_w1.to(dtype), weights.shared_w2.to(dtype), activation)
    lb, z = aux_losses(logits, counts, k, aux_coeff, z_coeff, score_fn)
    return dict(out=out, aux=lb + z, lb=lb, z=z, logits=logits, ids=ids, weights=topw,
                counts=counts, offsets=offsets, src_row=src, dest=dest)


def reference_eager_forward(x, weights, k, *, score_fn=SOFTMAX, activation=SWIGLU,
                            aux_coeff=0.01, z_coeff=0.001):
    """The reference's eager CPU layer written with torch's own ops, as RoutedFFN runs it
    (reference_blocks.py:35-45): fp32 rows, router F.linear (+ bias), logits.topk(k), softmax
    over the selected (sigmoid normalised over them for the sigmoid score), the shared expert
    first, then per expert torch.where over the top-k indices, the expert's FFN on the gathered
    rows weighted after fc2, and index_add into the output; the aux / z losses in closed form on
    the full logits (megatron_moe.py:44-45). Used as the timed CPU baseline; tie order is
    torch.topk's."""
    rows = x.detach().cpu().float()
    logits = F.linear(rows, weights.router.float())
    if weights.bias is not None:
        logits = logits + weights.bias.float()
    top, idx = logits.topk(k)
    if score_fn == SOFTMAX:
        w = top.softmax(-1)
    else:
        s = torch.sigmoid(top)
        w = s / s.sum(-1, keepdim=True)
    if weights.shared_w1 is not None:
        out = expert_ffn(rows, weights.shared_w1.float(), weights.shared_w2.float(), activation)
    else:
        out = torch.zeros_like(rows)
    for e in range(weights.router.shape[0]):
        token, slot = torch.where(idx == e)
        if token.numel():
            y = expert_ffn(rows[token], weights.w1[e].float(), weights.w2[e].float(), activation)
            out = out.index_add(0, token, y * w[token, slot, None])
    counts = torch.bincount(idx.flatten(), minlength=weights.router.shape[0])
    lb, z = aux_losses(logits, counts, k, aux_coeff, z_coeff, score_fn)
    return out, lb + z


def moe_forward_tokens(x, weights, k, tokens, *, logits, score_fn=SOFTMAX, activation=SWIGLU,
                       dtype=torch.float32):
    """Output rows for a subset of tokens only (every token's output depends on its own row and
    routing alone); used to check full-size runs without the full expert cost."""
    x = x.detach().cpu()
    tokens = torch.as_tensor(tokens, dtype=torch.long)
    ids, topw = topk(logits[tokens], k, score_fn)
    rows = x[tokens].to(dtype)
    out = torch.zeros_like(rows)
    for e in torch.unique(ids).tolist():
        tok, slot = torch.where(ids.long() == e)
        y = expert_ffn(rows[tok], weights.w1[e].to(dtype), weights.w2[e].to(dtype), activation)
        out.index_add_(0, tok, y * topw[tok, slot, None].to(dtype))
    if weights.shared_w1 is not None:
        out = out + expert_ffn(rows, weights.shared_w1.to(dtype), weights.shared_w2.to(dtype), activation)
    return out


# ---------------------------------------------------------------------------------------------
# fp8 (OCP e4m3fn) helpers: the quantisation the fp8 path applies and its dequantised reference.

def e4m3_round(v):
    """Round fp32 values (|v| <= 448) to e4m3fn with round-to-nearest-even; returns uint8 codes."""
    return v.float().to(torch.float8_e4m3fn).view(torch.uint8)


def e4m3_decode(codes):
    return codes.view(torch.float8_e4m3fn).float()


def quantize_rowwise(x):
    """Per-row e4m3: scale = amax(|row|) / 448 (1 for an all-zero row); q = e4m3(row / scale)."""
    x = x.float()
    amax = x.abs().amax(-1, keepdim=True)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    return e4m3_round(x / scale), scale.squeeze(-1)


def quantize_blockwise(w, block=128):
    """Per 128x128 block e4m3 of w [..., R, C] (R, C multiples of 128); scales [..., R/128, C/128]."""
    w = w.float()
    *lead, R, C = w.shape
    blocks = w.reshape(*lead, R // block, block, C // block, block)
    amax = blocks.abs().amax(dim=(-3, -1))
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = e4m3_round(blocks / scale[..., :, None, :, None]).reshape(*lead, R, C)
    return q, scale


def dequantize_blockwise(q, scale, block=128):
    *lead, R, C = q.shape
    v = e4m3_decode(q).reshape(*lead, R // block, block, C // block, block)
    return (v * scale[..., :, None, :, None]).reshape(*lead, R, C)


def dequantize_rowwise(q, scale):
    return e4m3_decode(q) * scale.float()[:, None]


def _fp8_expert(rows, w1q, w1s, w2q, w2s, activation):
    """fc1 on dequantised operands in fp32, activation, h rounded to bf16 and re-quantised per
    row, fc2 on dequantised operands."""
    w1 = dequantize_blockwise(w1q.cpu(), w1s.cpu())
    w2 = dequantize_blockwise(w2q.cpu(), w2s.cpu())
    h = act(rows @ w1.t(), activation, w2q.shape[-1]).to(torch.bfloat16).float()
    hq, hs = quantize_rowwise(h)
    return dequantize_rowwise(hq, hs) @ w2.t()


def moe_forward_fp8(x, router, w1q, w1s, w2q, w2s, k, *, score_fn=SOFTMAX, activation=SWIGLU,
                    aux_coeff=0.01, z_coeff=0.001, bias=None, tokens=None, shared=None):
    """The fp8 layer on the CPU, the fp32 dequantised reference of the fp8 path.

    Routing as moe_forward (fp32 router on the bf16 hidden states). Each token row is quantised
    per row to e4m3 (quantize_rowwise) and dequantised; expert weights are the dequantised
    128 x 128-block e4m3 weights; fc1 and the activation run in fp32, h is rounded to bf16 (the
    dtype the GPU path stores it in), quantised per row, dequantised, and fc2 runs in fp32;
    outputs are weighted after fc2 and accumulated in ascending expert order.
    The weight tensors may live on any device; only the experts in use are copied to the CPU.
    With `tokens`, out holds only those tokens' rows (each token's output depends on its own
    row and routing alone). `shared` = (w1q, w1s, w2q, w2s) of an always-on shared expert
    ([Fs, d], [d, Hs] matrices), added to every token.
    """
    x = x.detach().cpu()
    logits = router_logits_fixed(x, router, bias)
    E = router.shape[0]
    ids, topw = topk(logits, k, score_fn)
    counts, offsets, src, dest = route_plan(ids, E)
    xq, xs = quantize_rowwise(x.float())
    sel = torch.arange(x.shape[0]) if tokens is None else torch.as_tensor(tokens, dtype=torch.long)
    rows = dequantize_rowwise(xq[sel], xs[sel])
    out = torch.zeros(len(sel), x.shape[1], dtype=torch.float32)
    ids64 = ids.long()[sel]
    topw_sel = topw[sel]
    for e in range(E):
        token, slot = torch.where(ids64 == e)
        if not token.numel():
            continue
        y = _fp8_expert(rows[token], w1q[e], w1s[e], w2q[e], w2s[e], activation)
        out.index_add_(0, token, y * topw_sel[token, slot, None])
    if shared is not None:
        out = out + _fp8_expert(rows, *shared, activation)
    lb, z = aux_losses(logits, counts, k, aux_coeff, z_coeff, score_fn)
    return dict(out=out, aux=lb + z, lb=lb, z=z, logits=logits, ids=ids, weights=topw,
                counts=counts, offsets=offsets, src_row=src, dest=dest, x_q=xq, x_scale=xs)
