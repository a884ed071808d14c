"""Pins of the CPU oracle (CPU only): each oracle function is checked against something that
does not restate it -- the reference's own torch expression, exact arithmetic, brute force on
tiny inputs, hand-computed closed forms, or invariants -- chosen so that a dropped term, a wrong
index or sign, or a swapped operand fails at least one check.

Reference anchors: router logits F.linear(x.float(), W.float()) (megatron_moe.py:95-99,
reference_blocks.py:37); top-k then softmax over the selected (reference_blocks.py:37-38);
the mapping.T.nonzero() permutation and mapping.sum(0) counts (megatron_moe.py:142-144);
SwiGLU / ReLU^2 experts (megatron_moe.py:23-24, lm.py:29-35); routed mixture plus shared
expert (tests/test_scaling_reference_blocks.py:14-28); aux / z-loss closed forms.
"""
from fractions import Fraction
import math

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import moe_oracle as orc


def _bf16_ints(shape, lo, hi, g):
    return torch.randint(lo, hi, shape, generator=g).to(torch.bfloat16)


# ---------------------------------------------------------------------------------------------
# router logits

def test_fixed_order_logits_equal_f_linear_on_exact_data():
    """Small integers: every partial sum is exact in fp32, so any summation order -- the
    oracle's fixed one and torch's BLAS one -- must give identical bits."""
    g = torch.Generator().manual_seed(0)
    x = _bf16_ints((37, 300), -8, 9, g)
    w = torch.randint(-16, 17, (11, 300), generator=g).float()
    fixed = orc.router_logits_fixed(x, w)
    ref = orc.router_logits_reference(x, w)
    exact = (x.long() @ w.long().t()).float()
    assert torch.equal(ref, exact)
    assert torch.equal(fixed, exact)
    bias = torch.randint(-5, 6, (11,), generator=g).float()
    assert torch.equal(orc.router_logits_fixed(x, w, bias), exact + bias)


def test_fixed_order_logits_within_rounding_bound_of_fp64():
    """Recursive summation of n products has error <= gamma_n * sum |x_i w_i|
    (gamma_n = n u / (1 - n u), u = 2^-24): the oracle must sit inside that bound of the
    float64 dot product, and so must torch's F.linear."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    w = torch.randn(32, 1024, generator=g) * 0.02
    exact = x.double() @ w.double().t()
    mag = x.double().abs() @ w.double().abs().t()
    n, u = 1024, 2.0 ** -24
    bound = n * u / (1 - n * u) * mag
    for got in (orc.router_logits_fixed(x, w), orc.router_logits_reference(x, w)):
        assert ((got.double() - exact).abs() <= bound).all()


def _round_f32(q: Fraction) -> Fraction:
    """Correct round-to-nearest-even of an exact rational to float32."""
    f = np.float32(float(q))
    cands = {Fraction(float(f)),
             Fraction(float(np.nextafter(f, np.float32(np.inf)))),
             Fraction(float(np.nextafter(f, np.float32(-np.inf))))}
    best = min(cands, key=lambda c: (abs(c - q), c))
    ties = [c for c in cands if abs(c - q) == abs(best - q)]
    if len(ties) > 1:  # halfway: take the even mantissa
        ties.sort()
        best = next(c for c in ties
                    if int(np.float32(float(c)).view(np.uint32)) % 2 == 0)
    return best


def test_fixed_order_logits_match_exact_arithmetic_restatement():
    """The documented order, evaluated in exact rationals with one correct float32 rounding per
    fused multiply-add and per addition: chunks of 128 features, an FMA chain from 0 inside a
    chunk, chunk sums added left to right, bias last. Inputs span many binades so that a
    different chunking or order changes the bits."""
    g = torch.Generator().manual_seed(2)
    T, d, E = 3, 300, 4
    x = (torch.randn(T, d, generator=g) * torch.exp2(torch.randint(-6, 7, (T, d), generator=g))
         ).to(torch.bfloat16)
    w = torch.randn(E, d, generator=g) * torch.exp2(torch.randint(-12, 3, (E, d), generator=g)).float()
    bias = torch.randn(E, generator=g)
    got = orc.router_logits_fixed(x, w, bias)
    xf = x.float()

    def restated(t, e, chunk):
        total = None
        for c0 in range(0, d, chunk):
            acc = Fraction(0)
            for i in range(c0, min(c0 + chunk, d)):
                acc = _round_f32(Fraction(float(xf[t, i])) * Fraction(float(w[e, i])) + acc)
            total = acc if total is None else _round_f32(total + acc)
        return float(_round_f32(total + Fraction(float(bias[e]))))

    for t in range(T):
        for e in range(E):
            assert float(got[t, e]) == restated(t, e, 128), (t, e)
    # the check has teeth: another chunking changes some of these bits
    assert any(float(got[t, e]) != restated(t, e, 64) for t in range(T) for e in range(E))


# ---------------------------------------------------------------------------------------------
# top-k and weights

def _brute_topk(row, k):
    order = sorted(range(len(row)), key=lambda e: (-float(row[e]), e))
    return order[:k]


@pytest.mark.parametrize("E,k", [(1, 1), (4, 4), (8, 2), (13, 5), (64, 8), (256, 8)])
def test_topk_brute_force_with_ties(E, k):
    g = torch.Generator().manual_seed(E * 10 + k)
    # values from a small set so that ties are everywhere, including -0.0 against +0.0
    pool = torch.tensor([-1.5, -0.0, 0.0, 0.25, 0.25, 2.0, 3.0])
    logits = pool[torch.randint(0, len(pool), (50, E), generator=g)]
    ids, w = orc.topk(logits, k)
    for t in range(logits.shape[0]):
        assert ids[t].tolist() == _brute_topk(logits[t], k), t
    sel = torch.gather(logits.double(), 1, ids.long())
    assert torch.allclose(w.double(), sel.softmax(-1), rtol=1e-6, atol=0)


def test_topk_matches_torch_topk_without_ties():
    """Distinct logits: the reference's own ops (topk, softmax over the selected values)."""
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(200, 32, generator=g)
    ids, w = orc.topk(logits, 4)
    vals, idx = logits.topk(4)
    assert torch.equal(ids.long(), idx)
    assert torch.allclose(w, vals.softmax(-1), rtol=2e-6, atol=0)
    # softmax over the top-k == full softmax renormalised over the top-k
    p = logits.double().softmax(-1)
    sel = torch.gather(p, 1, idx)
    assert torch.allclose(w.double(), sel / sel.sum(-1, keepdim=True), rtol=1e-6, atol=0)


def test_sigmoid_weights_normalised_over_selected():
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(100, 128, generator=g)
    ids, w = orc.topk(logits, 8, orc.SIGMOID)
    vals, idx = logits.topk(8)
    assert torch.equal(ids.long(), idx)
    s = torch.sigmoid(vals.double())
    assert torch.allclose(w.double(), s / s.sum(-1, keepdim=True), rtol=1e-6, atol=0)
    assert torch.allclose(w.double().sum(-1), torch.ones(100, dtype=torch.float64), atol=1e-6)


# ---------------------------------------------------------------------------------------------
# route plan

def _reference_plan(ids, E):
    """megatron_moe.py:142-144 on a routing map built from ids."""
    T, k = ids.shape
    mapping = torch.zeros(T, E, dtype=torch.bool)
    mapping.scatter_(1, ids.long(), True)
    order = mapping.T.nonzero(as_tuple=False)[:, 1]
    counts = mapping.sum(0)
    return order, counts


@pytest.mark.parametrize("T,E,k", [(1, 4, 1), (7, 8, 8), (300, 16, 4), (64, 256, 8), (5, 3, 2)])
def test_route_plan_is_mapping_nonzero_order(T, E, k):
    g = torch.Generator().manual_seed(T + E + k)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()
    counts, offsets, src, dest = orc.route_plan(ids, E)
    order, ref_counts = _reference_plan(ids, E)
    assert torch.equal(src.long(), order)
    assert torch.equal(counts.long(), ref_counts)
    assert offsets[0] == 0 and torch.equal(offsets[1:].long(), ref_counts.cumsum(0))
    assert int(counts.sum()) == T * k
    # dest inverts src: assignment (t, j) lands on a row of expert ids[t, j] holding token t
    for t in range(T):
        for j in range(k):
            r = int(dest[t, j])
            assert int(src[r]) == t
            e = int(ids[t, j])
            assert offsets[e] <= r < offsets[e + 1]


def test_route_plan_empty_experts():
    ids = torch.tensor([[3, 1], [1, 3], [3, 1]], dtype=torch.int32)
    counts, offsets, src, _ = orc.route_plan(ids, 6)
    assert counts.tolist() == [0, 3, 0, 3, 0, 0]
    assert offsets.tolist() == [0, 0, 3, 3, 6, 6, 6]
    assert src.tolist() == [0, 1, 2, 0, 1, 2]


# ---------------------------------------------------------------------------------------------
# aux losses

def test_aux_hand_computed_example():
    """T=2, E=2, k=1, both tokens with logits [0, log 3]: s = [1/4, 3/4] per token, both go to
    expert 1, counts [0, 2]: lb = c * 2 / (1 * 4) * (3/2 * 2) = 1.5 c; lse = log 4."""
    logits = torch.tensor([[0.0, math.log(3)], [0.0, math.log(3)]])
    lb, z = orc.aux_losses(logits, torch.tensor([0, 2]), 1, 0.01, 0.001)
    # log 3 enters as an fp32 logit: 1e-7 relative is its rounding, not the formula
    assert lb == pytest.approx(0.015, rel=1e-7)
    assert z == pytest.approx(0.001 * math.log(4) ** 2, rel=1e-7)


def test_aux_uniform_router_gives_coefficient():
    """Uniform scores make sum_t s_te = T / E for every e, so lb = coeff whatever the counts."""
    for E, k, T in [(8, 2, 16), (32, 4, 100), (128, 8, 3)]:
        logits = torch.zeros(T, E)
        ids, _ = orc.topk(logits, k)
        counts, *_ = orc.route_plan(ids, E)
        lb, z = orc.aux_losses(logits, counts, k, 0.01, 0.001)
        assert lb == pytest.approx(0.01, rel=1e-12)
        assert z == pytest.approx(0.001 * math.log(E) ** 2, rel=1e-12)
        lb_s, _ = orc.aux_losses(logits, counts, k, 0.01, 0.001, orc.SIGMOID)
        assert lb_s == pytest.approx(0.01, rel=1e-12)


def test_aux_is_token_order_invariant_and_linear_in_coefficients():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(50, 16, generator=g)
    ids, _ = orc.topk(logits, 4)
    counts, *_ = orc.route_plan(ids, 16)
    lb, z = orc.aux_losses(logits, counts, 4, 0.01, 0.001)
    perm = torch.randperm(50, generator=g)
    lb2, z2 = orc.aux_losses(logits[perm], counts, 4, 0.01, 0.001)
    assert lb == pytest.approx(lb2, rel=1e-12) and z == pytest.approx(z2, rel=1e-12)
    lb3, z3 = orc.aux_losses(logits, counts, 4, 0.03, 0.002)
    assert lb3 == pytest.approx(3 * lb, rel=1e-12) and z3 == pytest.approx(2 * z, rel=1e-12)


# ---------------------------------------------------------------------------------------------
# experts and the layer

def test_swiglu_gate_is_the_first_half():
    """One unit, one feature: fc1 rows (gate a, value b); out = w2 * silu(a x) * (b x)."""
    x = torch.tensor([[1.0]])
    w1 = torch.tensor([[2.0], [3.0]])
    w2 = torch.tensor([[1.0]])
    out = orc.expert_ffn(x, w1, w2, orc.SWIGLU)
    assert out.item() == pytest.approx(F.silu(torch.tensor(2.0)).item() * 3.0, rel=1e-6)
    assert out.item() != pytest.approx(F.silu(torch.tensor(3.0)).item() * 2.0, rel=1e-3)


def test_relu2_expert_is_flexible_mlp():
    """lm.py:29-35: c_proj(relu(c_fc x)^2)."""
    g = torch.Generator().manual_seed(6)
    x, w1, w2 = torch.randn(9, 16, generator=g), torch.randn(8, 16, generator=g), torch.randn(16, 8, generator=g)
    ref = F.linear(F.relu(F.linear(x, w1)).square(), w2)
    assert torch.allclose(orc.expert_ffn(x, w1, w2, orc.RELU2), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("activation,score_fn", [(orc.SWIGLU, orc.SOFTMAX), (orc.RELU2, orc.SIGMOID)])
def test_layer_is_the_dense_weighted_mixture(activation, score_fn):
    """tests/test_scaling_reference_blocks.py:14-28: the routed layer equals the shared expert
    plus every expert applied densely, weighted by the top-k weights scattered into [T, E]."""
    g = torch.Generator().manual_seed(7)
    T, d, E, k, H = 40, 32, 6, 2, 16
    Fr = 2 * H if activation == orc.SWIGLU else H
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    wts = orc.Weights(router=torch.randn(E, d, generator=g) * 0.2,
                      w1=torch.randn(E, Fr, d, generator=g) * 0.2,
                      w2=torch.randn(E, d, H, generator=g) * 0.2,
                      shared_w1=torch.randn(Fr, d, generator=g) * 0.2,
                      shared_w2=torch.randn(d, H, generator=g) * 0.2)
    res = orc.moe_forward(x, wts, k, score_fn=score_fn, activation=activation, dtype=torch.float64)
    dense = torch.zeros(T, E, dtype=torch.float64).scatter(1, res["ids"].long(), res["weights"].double())
    xs = x.double()
    expected = orc.expert_ffn(xs, wts.shared_w1.double(), wts.shared_w2.double(), activation)
    for e in range(E):
        expected = expected + orc.expert_ffn(xs, wts.w1[e].double(), wts.w2[e].double(), activation) * dense[:, e, None]
    assert torch.allclose(res["out"], expected, rtol=1e-10, atol=1e-12)


def test_identical_experts_reduce_to_one_expert():
    """Normalised weights sum to one, so identical experts give exactly that expert's output."""
    g = torch.Generator().manual_seed(8)
    T, d, E, k, H = 30, 64, 8, 3, 32
    w1 = torch.randn(1, 2 * H, d, generator=g).expand(E, -1, -1)
    w2 = torch.randn(1, d, H, generator=g).expand(E, -1, -1)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    res = orc.moe_forward(x, orc.Weights(router=torch.randn(E, d, generator=g), w1=w1, w2=w2), k,
                          dtype=torch.float64)
    one = orc.expert_ffn(x.double(), w1[0].double(), w2[0].double(), orc.SWIGLU)
    assert torch.allclose(res["out"], one, rtol=1e-6, atol=1e-9)


# ---------------------------------------------------------------------------------------------
# fp8 e4m3 helpers

def _e4m3_value(code):
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return s * m / 8 * 2.0 ** -6
    return s * (1 + m / 8) * 2.0 ** (e - 7)


def test_e4m3_decode_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = orc.e4m3_decode(codes)
    for c in range(256):
        v = _e4m3_value(c)
        if math.isnan(v):
            assert math.isnan(got[c].item())
        else:
            assert got[c].item() == v, c
    assert orc.e4m3_decode(torch.tensor([0x7E], dtype=torch.uint8)).item() == 448.0


def test_e4m3_rowwise_and_blockwise_quantisation():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(16, 256, generator=g) * torch.exp2(torch.randint(-4, 5, (16, 1), generator=g)).float()
    x[3] = 0
    q, s = orc.quantize_rowwise(x)
    deq = orc.e4m3_decode(q) * s[:, None]
    assert s[3] == 1 and (deq[3] == 0).all()
    assert torch.allclose(orc.e4m3_decode(q).abs().amax(-1)[torch.arange(16) != 3],
                          torch.full((15,), 448.0))
    # round to nearest with 3 mantissa bits: relative error <= 2^-4 for normal codes
    big = orc.e4m3_decode(q).abs() >= 2.0 ** -6
    assert ((deq - x).abs()[big] <= (x.abs() * 2.0 ** -4)[big] + 1e-12).all()
    w = torch.randn(2, 256, 384, generator=g) * 0.02
    qb, sb = orc.quantize_blockwise(w)
    assert sb.shape == (2, 2, 3)
    back = orc.dequantize_blockwise(qb, sb)
    assert ((back - w).abs() <= w.abs() * 2.0 ** -4 + sb.amax() * 2.0 ** -9).all()


def test_fp8_layer_reduces_to_the_fp32_layer_on_dequantised_weights():
    """moe_forward_fp8 against moe_forward: with token rows that are e4m3 values whose row
    maximum is 448 (row scale 1, so quantising them is exact) and the dequantised 128 x 128-block
    weights as the fp32 layer's weights, the two differ only by the per-row e4m3 re-quantisation
    of h (relative error <= 2^-4 per element). Routing and aux are the same bits; a transposed or
    mis-scaled weight, a dropped term or a wrong expert order would miss the bound."""
    g = torch.Generator().manual_seed(21)
    T, d, E, k, H = 48, 256, 4, 2, 128
    codes = torch.randint(0, 256, (T, d), generator=g).to(torch.uint8)
    codes[(codes & 0x7F) >= 0x7E] = 0x38  # no NaN, nothing above 448 but the planted maximum
    x = orc.e4m3_decode(codes)
    x[:, 7] = 448.0
    x = x.to(torch.bfloat16)  # e4m3 values are exact in bf16
    router = torch.randn(E, d, generator=g) * 0.02
    w1q, w1s = orc.quantize_blockwise(torch.randn(E, 2 * H, d, generator=g) * 0.02)
    w2q, w2s = orc.quantize_blockwise(torch.randn(E, d, H, generator=g) * 0.02)
    fp8 = orc.moe_forward_fp8(x, router, w1q, w1s, w2q, w2s, k)
    xq, xs = orc.quantize_rowwise(x.float())
    assert (xs == 1).all() and torch.equal(orc.e4m3_decode(xq), x.float())
    ref = orc.moe_forward(x, orc.Weights(router=router, w1=orc.dequantize_blockwise(w1q, w1s),
                                         w2=orc.dequantize_blockwise(w2q, w2s)), k)
    assert torch.equal(fp8["ids"], ref["ids"]) and torch.equal(fp8["counts"], ref["counts"])
    assert fp8["aux"] == ref["aux"]
    err = ((fp8["out"] - ref["out"]).norm() / ref["out"].norm()).item()
    assert 1e-4 < err < 4e-2  # the h re-quantisation is visible, and bounded


# ---------------------------------------------------------------------------------------------
# committed golden vectors (written by tests/golden/make_golden.py) still reproduce

def test_oracle_reproduces_golden_vectors():
    from tests.golden_io import load_golden
    for name, case in load_golden().items():
        res = orc.moe_forward(case["x"], case["weights"], case["k"], score_fn=case["score_fn"],
                              activation=case["activation"])
        assert torch.equal(res["logits"].view(torch.int32), case["ref_logits"].view(torch.int32)), name
        for key in ("ids", "weights", "counts", "offsets", "src_row", "dest"):
            assert torch.equal(res[key], case["ref_" + key]), (name, key)
        assert torch.allclose(res["out"], case["ref_out"], rtol=1e-5, atol=1e-7), name
        assert np.allclose([res["aux"], res["lb"], res["z"]], case["ref_aux"], rtol=1e-12), name
    assert set(load_golden()) == {"ties", "sigmoid-relu2-shared-bias", "k-equals-E"}
    ties = load_golden()["ties"]
    assert torch.equal(ties["weights"].router[5], ties["weights"].router[3])


# ---------------------------------------------------------------------------------------------
# moe_forward_tokens (the reference of the full-size output checks) is moe_forward's rows

@pytest.mark.parametrize("activation,score_fn,shared,bias", [
    (orc.SWIGLU, orc.SOFTMAX, False, False),
    (orc.RELU2, orc.SOFTMAX, True, False),
    (orc.SWIGLU, orc.SIGMOID, True, True),
    (orc.RELU2, orc.SIGMOID, False, True),
])
def test_moe_forward_tokens_equals_moe_forward_rows(activation, score_fn, shared, bias):
    """Each token's output depends on its own row and routing alone, so the subset restatement
    must return exactly the full layer's rows, in the order asked for, for token lists that are
    unsorted, repeat tokens, or hold a single token. Run in float64: the expert products then
    carry no rounding that a different batch of rows could change."""
    g = torch.Generator().manual_seed(21)
    T, d, E, k, H = 96, 48, 7, 3, 24
    Fr = 2 * H if activation == orc.SWIGLU else H
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    wts = orc.Weights(router=torch.randn(E, d, generator=g) * 0.3,
                      w1=torch.randn(E, Fr, d, generator=g) * 0.2,
                      w2=torch.randn(E, d, H, generator=g) * 0.2,
                      shared_w1=torch.randn(Fr, d, generator=g) * 0.2 if shared else None,
                      shared_w2=torch.randn(d, H, generator=g) * 0.2 if shared else None,
                      bias=torch.randn(E, generator=g) if bias else None)
    full = orc.moe_forward(x, wts, k, score_fn=score_fn, activation=activation,
                           dtype=torch.float64)
    lists = [torch.randperm(T, generator=g)[:40],            # unsorted
             torch.tensor([5, 5, 90, 3, 5, 90, 0, T - 1]),   # duplicates
             torch.tensor([17]),
             torch.arange(T)]
    for tokens in lists:
        sub = orc.moe_forward_tokens(x, wts, k, tokens, logits=full["logits"], score_fn=score_fn,
                                     activation=activation, dtype=torch.float64)
        torch.testing.assert_close(sub, full["out"][tokens], rtol=1e-13, atol=1e-15)
    # discriminates: another token's row, or a dropped shared expert, is far off
    sub = orc.moe_forward_tokens(x, wts, k, lists[0], logits=full["logits"], score_fn=score_fn,
                                 activation=activation, dtype=torch.float64)
    assert not torch.allclose(sub, full["out"][lists[0].roll(1)], rtol=1e-3)
    if shared:
        no_shared = orc.Weights(router=wts.router, w1=wts.w1, w2=wts.w2, bias=wts.bias)
        sub = orc.moe_forward_tokens(x, no_shared, k, lists[0], logits=full["logits"],
                                     score_fn=score_fn, activation=activation,
                                     dtype=torch.float64)
        assert not torch.allclose(sub, full["out"][lists[0]], rtol=1e-3)


# ---------------------------------------------------------------------------------------------
# routing on the fixed-order logits equals routing on the reference's own router expression

@pytest.mark.parametrize("config", [1, 2, 3, 4, 5, 6])
def test_fixed_order_routing_equals_reference_router_at_benchmark_configs(config):
    """On the seeded inputs of every benchmark configuration, top-k of the fixed-order logits
    (which the HIP router reproduces bit for bit) selects the same experts in the same order as
    top-k of the reference's F.linear(x.float(), W.float()) (+ the logit bias)
    (megatron_moe.py:95-99, reference_blocks.py:37-38), although most logits differ in their
    low bits. The weights then differ only by that rounding. Reported: the smallest k-th /
    (k+1)-th logit margin, the largest logit difference of the two orders and the number of
    near-tie tokens whose margin is within twice their own difference."""
    from tests.moe_cases import CONFIGS, make_router_inputs
    case = CONFIGS[config]
    x, router, bias = make_router_inputs(case)
    fixed = orc.router_logits_fixed(x, router, bias)
    ref = orc.router_logits_reference(x, router, bias)
    assert (fixed != ref).any()  # the two orders do round differently
    ids_f, w_f = orc.topk(fixed, case.k, case.score_fn)
    ids_r, w_r = orc.topk(ref, case.k, case.score_fn)
    assert torch.equal(ids_f, ids_r)
    torch.testing.assert_close(w_f, w_r, rtol=1e-5, atol=1e-7)
    # Per token: the selection can only flip where the gap between the k-th and (k+1)-th logit
    # is within twice that token's largest difference between the two orders; those tokens
    # (near ties) are counted -- they select identically here too (asserted above).
    top = ref.double().sort(-1, descending=True).values
    margin_t = top[:, case.k - 1] - top[:, case.k]
    diff_t = (fixed.double() - ref.double()).abs().max(-1).values
    near = int((margin_t <= 2 * diff_t).sum())
    print(f"config {config}: min top-k margin {margin_t.min().item():.3e}, max |fixed - F.linear| "
          f"{diff_t.max().item():.3e}, near-tie tokens {near} of {case.T}")
    assert near <= case.T // 100  # near ties are rare: the id check is not vacuous


@pytest.mark.parametrize("activation,score_fn,shared", [
    (orc.SWIGLU, orc.SOFTMAX, False), (orc.RELU2, orc.SIGMOID, True)])
def test_reference_eager_forward_is_the_layer(activation, score_fn, shared):
    """The torch-ops CPU baseline computes the same layer as moe_forward with the reference
    router (distinct logits, so the tie order cannot matter)."""
    g = torch.Generator().manual_seed(41)
    T, d, E, k, H = 80, 32, 6, 2, 16
    Fr = 2 * H if activation == orc.SWIGLU else H
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    wts = orc.Weights(router=torch.randn(E, d, generator=g) * 0.3,
                      w1=torch.randn(E, Fr, d, generator=g) * 0.2,
                      w2=torch.randn(E, d, H, generator=g) * 0.2,
                      shared_w1=torch.randn(Fr, d, generator=g) * 0.2 if shared else None,
                      shared_w2=torch.randn(d, H, generator=g) * 0.2 if shared else None,
                      bias=torch.randn(E, generator=g))
    out, aux = orc.reference_eager_forward(x, wts, k, score_fn=score_fn, activation=activation)
    ref = orc.moe_forward(x, wts, k, score_fn=score_fn, activation=activation, router="reference")
    torch.testing.assert_close(out, ref["out"], rtol=1e-5, atol=1e-6)
    assert aux == pytest.approx(ref["aux"], rel=1e-12)
