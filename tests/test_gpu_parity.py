"""GPU parity of the HIP MoE forward against the CPU oracle, through the ntmoe ops (C ABI).

Bar: routing (top-k ids, per-expert counts, offsets, permutation order, combine order) is
bit-exact; logits are bit-exact to the fixed-order C restatement; outputs are within relative
L2 1e-2 of the fp32 reference computed from the same bf16 inputs and bf16-rounded weights.
"""
import pytest
import torch

from oracle import moe_oracle as orc
from tests.moe_cases import Case, make_inputs, make_router_inputs, rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2  # relative L2 against the fp32 reference

SMALL = [
    Case("cfg1-shape", 512, 256, 8, 2, 512),
    Case("ragged-T1000-E32-k4", 1000, 1024, 32, 4, 512, seed=1),
    Case("E128-k8-sigmoid", 300, 512, 128, 8, 256, score_fn=1, seed=2),
    Case("E64-k8-zipf", 777, 256, 64, 8, 128, zipf_bias=1.2, seed=3),
    Case("relu2-d1280-H320", 130, 1280, 16, 4, 320, activation=1, seed=4),
    Case("E256-k8-two-tokens", 2, 128, 256, 8, 64, seed=5),
    Case("shared-expert", 200, 256, 16, 2, 128, shared_H=256, seed=6),
    Case("single-token", 1, 64, 4, 1, 64, seed=7),
]

# Mid-size batches (256 64-token blocks on a 256-CU part): the split router's item order, plane
# layout and top-k at the sizes the benchmark configurations use, with a ragged last block.
MID = [
    Case("quarter-T16411-d512-E24-k3-bias", 16411, 512, 24, 3, 64, zipf_bias=1.2, seed=8),
    Case("quarter-T16400-d1024-E32-k4-sigmoid", 16400, 1024, 32, 4, 64, score_fn=1, seed=9),
]


def gpu_inputs(case):
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    return cpu, dict(
        x=cpu["x"].to(dev),
        wt=cpu["router"].t().contiguous().to(dev),
        w1=cpu["w1"].to(torch.bfloat16).to(dev),
        w2=cpu["w2"].to(torch.bfloat16).to(dev),
        sw1=None if cpu["shared_w1"] is None else cpu["shared_w1"].to(torch.bfloat16).to(dev),
        sw2=None if cpu["shared_w2"] is None else cpu["shared_w2"].to(torch.bfloat16).to(dev),
        bias=None if cpu["bias"] is None else cpu["bias"].to(dev),
    )


def oracle_weights(cpu):
    r = lambda t: None if t is None else t.to(torch.bfloat16).float()
    return orc.Weights(router=cpu["router"], w1=r(cpu["w1"]), w2=r(cpu["w2"]),
                       shared_w1=None if cpu["shared_w1"] is None else r(cpu["shared_w1"])[0],
                       shared_w2=None if cpu["shared_w2"] is None else r(cpu["shared_w2"])[0],
                       bias=cpu["bias"])


@pytest.mark.parametrize("case", SMALL + MID, ids=lambda c: c.name)
def test_router_logits_and_topk_bit_exact(case):
    from nexttransformer_amd import ops
    cpu, g = gpu_inputs(case)
    logits, ids, w, pp, zp = ops.router(g["x"], g["wt"], g["bias"], case.k, case.score_fn, True)
    torch.cuda.synchronize()
    ref_logits = orc.router_logits_fixed(cpu["x"], cpu["router"], cpu["bias"])
    ref_ids, ref_w = orc.topk(ref_logits, case.k, case.score_fn)
    assert torch.equal(logits.cpu().view(torch.int32), ref_logits.view(torch.int32)), "logits bits"
    assert torch.equal(ids.cpu(), ref_ids), "top-k ids"
    torch.testing.assert_close(w.cpu(), ref_w, rtol=2e-6, atol=2e-7)
    # aux partials against the closed forms
    s = orc.full_scores(ref_logits, case.score_fn)
    torch.testing.assert_close(pp.cpu().double().sum(0), s.sum(0), rtol=1e-5, atol=1e-5)
    lse2 = torch.logsumexp(ref_logits.double(), -1).square().sum()
    torch.testing.assert_close(zp.cpu().double().sum(), lse2, rtol=1e-5, atol=1e-5)


VARIANTS = ([(v, E, T, 1024) for v in ("no-buffers", "workspace", "logits-buffer")
             for E in (32, 64, 128) for T in (512, 4096)]
            # 5 and 10 chunks of 128 features: the fused and logits kernels split them over four
            # feature ranges of unequal length (1,1,1,2 and 2,3,2,3 chunks)
            + [(v, E, T, d) for d in (640, 1280) for v in ("no-buffers", "logits-buffer")
               for E in (32, 128) for T in (512, 4096)]
            + [(v, 256, 4096, d) for d in (640, 1280) for v in ("workspace", "logits-buffer")])


@pytest.mark.parametrize("variant,E,T,d", VARIANTS, ids=lambda v: str(v))
def test_router_variants_bit_exact_via_abi(variant, E, T, d):
    """Raw C-ABI calls that reach each router kernel (on a 256-CU part): with neither workspace
    nor a logits buffer the fused kernel (top-k in the block; one, two and four expert blocks);
    with the workspace the chunk planes (T = 512) or the logits kernel + top-k (T = 4096); with
    only a logits buffer the logits kernel. All follow the same order: identical bits."""
    import ctypes
    from nexttransformer_amd import _native as nat
    case = Case("variant", T, d, E, 4, 64, seed=11)
    cpu, g = gpu_inputs(case)
    lib = nat.load()
    d, k = case.d, case.k
    nblk = (T + 63) // 64
    logits = torch.empty(T, E, device="cuda")
    ids = torch.empty(T, k, device="cuda", dtype=torch.int32)
    w = torch.empty(T, k, device="cuda")
    pp = torch.empty(nblk, E, device="cuda")
    zp = torch.empty(nblk, device="cuda")
    need = lib.nt_moe_router_workspace_bytes(T, d, E, k)
    ws = torch.empty(max(need, 1), device="cuda", dtype=torch.uint8)
    use_ws = variant == "workspace"
    use_logits = variant != "no-buffers"
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = lib.nt_moe_router_fwd(nat.ptr(g["x"]), d, nat.ptr(g["wt"]), None, T, d, E, k, 0,
                               nat.ptr(logits) if use_logits else None, nat.ptr(ids), nat.ptr(w),
                               nat.ptr(pp), nat.ptr(zp), nat.ptr(ws) if use_ws else None,
                               need if use_ws else 0, stream)
    nat.check(st, "router")
    torch.cuda.synchronize()
    ref_logits = orc.router_logits_fixed(cpu["x"], cpu["router"])
    if use_logits:
        assert torch.equal(logits.cpu().view(torch.int32), ref_logits.view(torch.int32))
    ref_ids, ref_w = orc.topk(ref_logits, k)
    assert torch.equal(ids.cpu(), ref_ids)
    torch.testing.assert_close(w.cpu(), ref_w, rtol=2e-6, atol=2e-7)
    s_ = orc.full_scores(ref_logits, 0)
    torch.testing.assert_close(pp.cpu().double().sum(0), s_.sum(0), rtol=1e-5, atol=1e-5)


# The streamed router (129-256 experts, at least 64 token blocks): E not a multiple of 32, a
# partial last 64-feature stage (d = 1032) and a one-chunk d, a ragged last token block, bias,
# sigmoid, top-6 and top-8.
STREAM = [
    Case("stream-T4100-d1032-E200-k8-sigmoid-bias", 4100, 1032, 200, 8, 64, score_fn=1,
         zipf_bias=0.8, seed=21),
    Case("stream-T4096-d1280-E256-k8", 4096, 1280, 256, 8, 64, seed=22),
    Case("stream-T4160-d264-E160-k6-bias", 4160, 264, 160, 6, 64, zipf_bias=1.2, seed=23),
]


@pytest.mark.parametrize("case", STREAM, ids=lambda c: c.name)
def test_streamed_router_bit_exact(case):
    from nexttransformer_amd import ops
    x, router, bias = make_router_inputs(case)
    dev = torch.device("cuda")
    logits, ids, w, pp, zp = ops.router(x.to(dev), router.t().contiguous().to(dev),
                                        None if bias is None else bias.to(dev), case.k,
                                        case.score_fn, True)
    torch.cuda.synchronize()
    ref_logits = orc.router_logits_fixed(x, router, bias)
    assert torch.equal(logits.cpu().view(torch.int32), ref_logits.view(torch.int32)), "logits bits"
    ref_ids, ref_w = orc.topk(ref_logits, case.k, case.score_fn)
    assert torch.equal(ids.cpu(), ref_ids), "top-k ids"
    torch.testing.assert_close(w.cpu(), ref_w, rtol=2e-6, atol=2e-7)
    s_ = orc.full_scores(ref_logits, case.score_fn)
    torch.testing.assert_close(pp.cpu().double().sum(0), s_.sum(0), rtol=1e-5, atol=1e-5)
    lse2 = torch.logsumexp(ref_logits.double(), -1).square().sum()
    torch.testing.assert_close(zp.cpu().double().sum(), lse2, rtol=1e-5, atol=1e-5)


# router_plan (router + plan in one call, the router's top-k counting each 64-token block's
# assignments): the chunk-per-wave kernel (E <= 32, d <= 1024), the fused range, logits + top-k
# and planes paths, the streamed kernel, ragged last blocks, E not dividing 256, and the T3 cell.
ROUTER_PLAN = SMALL + MID + STREAM + [
    Case("t3-T16384-d1280-E256-k8", 16384, 1280, 256, 8, 64, seed=24),
    Case("E64-T16400-d2048-k8-zipf", 16400, 2048, 64, 8, 64, zipf_bias=1.2, seed=25),
    Case("E128-T8192-d2048-k8-sigmoid", 8192, 2048, 128, 8, 64, score_fn=1, seed=26),
]


@pytest.mark.parametrize("case", ROUTER_PLAN, ids=lambda c: c.name)
def test_router_plan_equals_router_then_route_plan(case):
    """Every output of the one-call router + plan bit-identical to router followed by
    route_plan (the histogram path), on the same inputs."""
    from nexttransformer_amd import ops
    x, router, bias = make_router_inputs(case)
    dev = torch.device("cuda")
    x, wt = x.to(dev), router.t().contiguous().to(dev)
    bias = None if bias is None else bias.to(dev)
    ref = ops.router(x, wt, bias, case.k, case.score_fn, True)
    ref = ref + ops.route_plan(ref[1], ref[2], case.E, None, False)[:6]
    got = ops.router_plan(x, wt, bias, case.k, case.score_fn, True)
    torch.cuda.synchronize()
    names = ("logits", "ids", "weights", "prob_partial", "z_partial", "counts", "offsets",
             "src_row", "perm_w", "combine_dest", "combine_w")
    for name, a, b in zip(names, got, ref):
        assert a.shape == b.shape, name
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
    assert int(got[5].sum()) == case.T * case.k


def test_router_plan_empty_batch():
    from nexttransformer_amd import ops
    dev = torch.device("cuda")
    x = torch.empty(0, 256, device=dev, dtype=torch.bfloat16)
    wt = torch.randn(256, 16, device=dev)
    out = ops.router_plan(x, wt, None, 2, 0, False)
    torch.cuda.synchronize()
    assert out[1].shape == (0, 2) and out[7].shape == (0,)
    assert torch.equal(out[5].cpu(), torch.zeros(16, dtype=torch.int32))
    assert torch.equal(out[6].cpu(), torch.zeros(17, dtype=torch.int32))


def test_topk_on_reference_logits_and_ties():
    """Top-k on the reference's own F.linear logits, plus constructed ties (lower index wins)."""
    from nexttransformer_amd import ops
    case = Case("ref-logits", 2048, 512, 32, 4, 64, seed=12)
    cpu = make_inputs(case)
    logits = orc.router_logits_reference(cpu["x"], cpu["router"])
    logits[:64] = 0.0                        # all tied: ids 0..k-1
    logits[64:128, ::2] = 1.0                # pairs of ties
    logits[128:192] = torch.randint(0, 3, (64, 32)).float()  # many ties
    logits[192:256, 5] = float("-0.0")
    for score_fn in (0, 1):
        ids, w, _, _ = ops.topk_from_logits(logits.cuda(), case.k, score_fn)
        ref_ids, ref_w = orc.topk(logits, case.k, score_fn)
        assert torch.equal(ids.cpu(), ref_ids)
        torch.testing.assert_close(w.cpu(), ref_w, rtol=2e-6, atol=2e-7)
    assert ids[:64].cpu().tolist() == [[0, 1, 2, 3]] * 64


def test_topk_256_experts_threshold_path_and_ties():
    """256 experts, top-8: 16 logits per lane, where the top-k inserts only the logits at or
    above the smallest lane maximum. Constructed rows: all tied, ties in pairs, many ties, the
    whole top 8 in one lane's share (experts 16 i), -0.0 beside +0.0, -inf everywhere but a few
    experts, and the reference's own logits."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(21)
    T, E, k = 512, 256, 8
    x = torch.randn(T, 256, generator=gen).to(torch.bfloat16)
    w = torch.randn(E, 256, generator=gen) * 0.05
    logits = orc.router_logits_reference(x, w)
    logits[:64] = 0.0
    logits[64:128, ::2] = 1.0
    logits[128:192] = torch.randint(0, 3, (64, E), generator=gen).float()
    logits[192:256] = -1.0
    logits[192:256, 0:256:16] = 10.0 + torch.arange(16).float()  # one lane's share
    logits[256:320] = 0.0
    logits[256:320, 1::2] = float("-0.0")
    logits[320:384] = float("-inf")
    logits[320:384, 7] = 1.0
    logits[320:384, 200] = 2.0
    for score_fn in (0, 1):
        ids, wts, _, _ = ops.topk_from_logits(logits.cuda(), k, score_fn)
        ref_ids, ref_w = orc.topk(logits, k, score_fn)
        assert torch.equal(ids.cpu(), ref_ids)
        torch.testing.assert_close(wts.cpu(), ref_w, rtol=2e-6, atol=2e-7)
    assert ids[:64].cpu().tolist() == [list(range(8))] * 64
    assert ids[192:256].cpu().tolist() == [[16 * i for i in range(15, 7, -1)]] * 64


@pytest.mark.parametrize("case", SMALL, ids=lambda c: c.name)
def test_route_plan_bit_exact(case):
    from nexttransformer_amd import ops
    cpu, g = gpu_inputs(case)
    _, ids, w, _, _ = ops.router(g["x"], g["wt"], g["bias"], case.k, case.score_fn, False)
    counts, offsets, src, perm_w, cdest, cw, x_perm = ops.route_plan(ids, w, case.E, g["x"], True)
    torch.cuda.synchronize()
    ids_c = ids.cpu()
    r_counts, r_offsets, r_src, r_dest = orc.route_plan(ids_c, case.E)
    assert torch.equal(counts.cpu(), r_counts)
    assert torch.equal(offsets.cpu(), r_offsets)
    assert torch.equal(src.cpu(), r_src)
    # reference expression: ids = mapping.T.nonzero()[:, 1] (megatron_moe.py:142)
    mapping = torch.zeros(case.T, case.E, dtype=torch.bool)
    mapping[torch.arange(case.T)[:, None], ids_c.long()] = True
    assert torch.equal(src.cpu().long(), mapping.T.nonzero()[:, 1])
    # combine order: ascending expert per token
    order = ids_c.long().argsort(-1)
    assert torch.equal(cdest.cpu(), r_dest.gather(1, order.int().long()))
    torch.testing.assert_close(cw.cpu(), w.cpu().gather(1, order))
    torch.testing.assert_close(perm_w.cpu()[r_dest.long()], w.cpu())
    assert torch.equal(x_perm.cpu(), cpu["x"][r_src.long()])


# (T, E, k, skew): the one-launch scan + permutation (counts table of ceil(T/256) x E entries up
# to 16384: the benchmark shapes, E not dividing 256, E = 256, a ragged last block) and the
# three-launch path beyond that table size (T = 40000, E = 128).
PLAN_SHAPES = [(1, 4, 1, 0.0), (1000, 32, 4, 0.0), (16384, 32, 4, 0.0), (32768, 64, 8, 1.2),
               (8192, 128, 8, 0.0), (300, 256, 8, 0.0), (777, 96, 3, 1.2), (16411, 24, 3, 0.0),
               (40000, 128, 2, 1.2)]


@pytest.mark.parametrize("T,E,k,skew", PLAN_SHAPES)
def test_route_plan_one_call_matches_oracle_and_two_calls(T, E, k, skew):
    """nt_moe_route_plan (the module's path) against the oracle, the reference's
    mapping.T.nonzero() order, and nt_moe_histogram_scan + nt_moe_permute, bit for bit."""
    import ctypes
    from nexttransformer_amd import _native as nat, ops
    g = torch.Generator().manual_seed(T * 7 + E)
    scores = torch.rand(T, E, generator=g) - skew * torch.log1p(torch.arange(E).float())
    ids_c = scores.topk(k, dim=1).indices.int()
    w_c = torch.rand(T, k, generator=g)
    ids, w = ids_c.cuda(), w_c.cuda()
    counts, offsets, src, perm_w, cdest, cw, _ = ops.route_plan(ids, w, E, None, False)
    r_counts, r_offsets, r_src, r_dest = orc.route_plan(ids_c, E)
    assert torch.equal(counts.cpu(), r_counts)
    assert torch.equal(offsets.cpu(), r_offsets)
    assert torch.equal(src.cpu(), r_src)
    mapping = torch.zeros(T, E, dtype=torch.bool)
    mapping[torch.arange(T)[:, None], ids_c.long()] = True
    assert torch.equal(src.cpu().long(), mapping.T.nonzero()[:, 1])
    order = ids_c.long().argsort(-1)
    assert torch.equal(cdest.cpu(), r_dest.gather(1, order))
    assert torch.equal(cw.cpu(), w_c.gather(1, order))
    assert torch.equal(perm_w.cpu()[r_dest.long()], w_c)
    # the same outputs from the two separate entry points
    lib = nat.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ws_bytes = lib.nt_moe_route_workspace_bytes(T, k, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    c2, o2 = torch.empty_like(counts), torch.empty_like(offsets)
    s2, p2, d2, w2 = (torch.empty_like(src), torch.empty_like(perm_w), torch.empty_like(cdest),
                      torch.empty_like(cw))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.nt_moe_histogram_scan(P(ids), T, k, E, P(c2), P(o2), P(ws), ws_bytes, stream) == 0
    assert lib.nt_moe_permute(None, 0, P(ids), P(w), T, 0, k, E, P(ws), ws_bytes, P(s2), P(p2),
                              P(d2), P(w2), None, stream) == 0
    torch.cuda.synchronize()
    for a, b in ((counts, c2), (offsets, o2), (src, s2), (perm_w, p2), (cdest, d2), (cw, w2)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("case", SMALL, ids=lambda c: c.name)
@pytest.mark.parametrize("permute_rows", [False, True])
def test_layer_forward_matches_fp32_reference(case, permute_rows):
    from nexttransformer_amd import ops
    cpu, g = gpu_inputs(case)
    out, aux, state = ops.moe_forward(g["x"], g["wt"], g["w1"], g["w2"], top_k=case.k,
                                      score_fn=case.score_fn, activation=case.activation,
                                      logit_bias=g["bias"], shared_w1=g["sw1"],
                                      shared_w2=g["sw2"], permute_rows=permute_rows)
    torch.cuda.synchronize()
    ref = orc.moe_forward(cpu["x"], oracle_weights(cpu), case.k, score_fn=case.score_fn,
                          activation=case.activation)
    assert torch.equal(state["ids"].cpu(), ref["ids"])
    assert torch.equal(state["counts"].cpu(), ref["counts"])
    err = rel_l2(out.float(), ref["out"])
    assert err <= BF16_TOL, f"relative L2 {err:.3e}"
    torch.testing.assert_close(aux[1].item(), ref["lb"], rtol=1e-4, atol=1e-7)
    torch.testing.assert_close(aux[2].item(), ref["z"], rtol=1e-4, atol=1e-7)
    torch.testing.assert_close(aux[0].item(), ref["aux"], rtol=1e-4, atol=1e-7)


def test_forward_is_deterministic():
    from nexttransformer_amd import ops
    case = Case("det", 4096, 1024, 32, 4, 512, seed=13)
    _, g = gpu_inputs(case)
    runs = [ops.moe_forward(g["x"], g["wt"], g["w1"], g["w2"], top_k=case.k)[:2] for _ in range(3)]
    for out, aux in runs[1:]:
        assert torch.equal(out.view(torch.int16), runs[0][0].view(torch.int16))
        assert torch.equal(aux, runs[0][1])
