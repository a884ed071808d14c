"""GPU parity of the layer backward against fp32 autograd.

The reference is the layer written in plain PyTorch fp32 on the CPU (router GEMM, softmax or
sigmoid over the k selected, per-expert SwiGLU / ReLU^2 FFNs with the bf16-rounded weights the
forward uses, the shared expert, the MCore load-balance and z losses: megatron_moe.py:43-45,
137-150, reference_blocks.py:35-45), differentiated by autograd for
loss = <out, G> + g_aux * aux with a random G. The expert selection is the forward's (ids), so
ties cannot differ. Bar: relative L2 <= 2e-2 for every gradient (the GPU path keeps bf16
intermediates: the combine transpose, the recomputed fc1 pre-activations, dh, d fc1 and the
weight-gradient products are bf16 with fp32 accumulation).
"""
import pytest
import torch

from tests.moe_cases import Case, make_inputs, rel_l2

pytestmark = pytest.mark.gpu

TOL = 2e-2

CASES = [
    Case("bwd-T512-d256-E8-k2-swiglu", 512, 256, 8, 2, 128, seed=21),
    Case("bwd-T300-d512-E16-k4-sigmoid-shared", 300, 512, 16, 4, 256, score_fn=1, shared_H=256,
         seed=22),
    Case("bwd-T700-d256-E32-k8-relu2-zipf", 700, 256, 32, 8, 128, activation=1, zipf_bias=1.2,
         seed=23),
    Case("bwd-T1024-d1024-E32-k4-swiglu", 1024, 1024, 32, 4, 512, seed=24),
    # the registered T3 expert cell's widths (d 1280, ReLU^2 width 320, shared expert)
    Case("bwd-T200-d1280-E16-k4-relu2-H320-shared", 200, 1280, 16, 4, 320, activation=1,
         shared_H=320, seed=25),
    # the packed path with the kept pre-activations for ReLU^2 and for skewed routing
    Case("bwd-T700-d512-E32-k8-relu2-H256-zipf", 700, 512, 32, 8, 256, activation=1,
         zipf_bias=1.2, seed=26),
    Case("bwd-T600-d512-E24-k6-relu2-sigmoid-H256-shared", 600, 512, 24, 6, 256, activation=1,
         score_fn=1, shared_H=256, seed=27),
]


def _packable(case):
    """Whether every projection of the case qualifies for the packed GEMM."""
    from nexttransformer_amd import _native as nat, ops
    up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
    widths = [case.H] + ([case.shared_H] if case.shared_H else [])
    return all(ops.packable(case.d, h, up) and ops.packable(h, case.d, nat.EPI_NONE)
               for h in widths)


# (case, mode) pairs: every case with plain weights; the fc1 recompute on three of them; the
# packed variant where the widths allow
RUNS = ([(c, "plain") for c in CASES] + [(c, "recompute") for c in CASES[:2] + CASES[4:5]]
        + [(c, "packed") for c in CASES if _packable(c)])


def ffn(x, w1, w2, activation):
    f = x @ w1.t()
    if activation == 0:
        H = w2.shape[1]
        h = torch.nn.functional.silu(f[:, :H]) * f[:, H:]
    else:
        h = torch.relu(f).square()
    return h @ w2.t()


def reference_grads(x, wr, bias, w1, w2, sw1, sw2, ids, G, g_aux, case, aux_coeff, z_coeff):
    x = x.float().clone().requires_grad_()
    wr = wr.float().clone().requires_grad_()
    w1 = w1.to(torch.bfloat16).float().requires_grad_()
    w2 = w2.to(torch.bfloat16).float().requires_grad_()
    params = [x, wr, w1, w2]
    if sw1 is not None:
        sw1 = sw1.to(torch.bfloat16).float().requires_grad_()
        sw2 = sw2.to(torch.bfloat16).float().requires_grad_()
        params += [sw1, sw2]
    T, E, k = case.T, case.E, case.k
    logits = x @ wr.t()
    if bias is not None:
        logits = logits + bias
    ids = ids.long()
    sel = logits.gather(1, ids)
    if case.score_fn == 0:
        w = sel.softmax(-1)
    else:
        s = torch.sigmoid(sel)
        w = s / s.sum(-1, keepdim=True)
    out = torch.zeros(T, x.shape[1])
    for e in range(E):
        tok, slot = torch.where(ids == e)
        if tok.numel():
            out = out.index_add(0, tok, ffn(x[tok], w1[e], w2[e], case.activation) * w[tok, slot, None])
    if sw1 is not None:
        out = out + ffn(x, sw1[0], sw2[0], case.activation)
    counts = torch.bincount(ids.flatten(), minlength=E).float()
    if case.score_fn == 0:
        p = logits.softmax(-1)
    else:
        s = torch.sigmoid(logits)
        p = s / s.sum(-1, keepdim=True)
    lb = aux_coeff * E / (k * T * T) * (p.sum(0) * counts).sum()
    z = z_coeff * torch.logsumexp(logits, -1).square().mean()
    loss = (out * G).sum() + g_aux * (lb + z)
    loss.backward()
    return [t.grad for t in params]


@pytest.mark.parametrize("case,mode", RUNS, ids=[f"{c.name}-{m}" for c, m in RUNS])
def test_backward_matches_fp32_autograd(case, mode):
    """packed: the forward runs the packed GEMMs; plain: the plain-weight GEMMs. Both keep the
    fc1 pre-activations from the up projection's launch (the module's training path);
    recompute: the plain forward's kept fc1 (routed and shared) is dropped, so the backward
    recomputes it."""
    from nexttransformer_amd import _native as nat, ops
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    aux_coeff, z_coeff, g_aux = 0.01, 0.001, 3.0
    x = cpu["x"].to(dev)
    wr = cpu["router"]  # fp32 [E, d]
    wr_t = wr.t().contiguous().to(dev)
    bias = None if cpu["bias"] is None else cpu["bias"].to(dev)
    bf = torch.bfloat16
    w1b, w2b = cpu["w1"].to(bf).to(dev), cpu["w2"].to(bf).to(dev)
    sw1b = sw2b = None
    if cpu["shared_w1"] is not None:
        sw1b, sw2b = cpu["shared_w1"].to(bf).to(dev), cpu["shared_w2"].to(bf).to(dev)
    fw = dict(w1=w1b, w2=w2b, shared_w1=sw1b, shared_w2=sw2b)
    packed = mode == "packed"
    if packed:
        up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
        fw = {n: None if w is None else ops.pack_expert_weights(w, up if "1" in n else nat.EPI_NONE)
              for n, w in fw.items()}
    out, aux, state = ops.moe_forward(x, wr_t, fw["w1"], fw["w2"], top_k=case.k,
                                      score_fn=case.score_fn, activation=case.activation,
                                      aux_coeff=aux_coeff, z_coeff=z_coeff, logit_bias=bias,
                                      shared_w1=fw["shared_w1"], shared_w2=fw["shared_w2"],
                                      want_logits=True, keep=True, packed=packed)
    assert state["fc1"] is not None
    assert (state["shared_fc1"] is not None) == (case.shared_H > 0)
    if mode == "recompute":
        state["fc1"] = state["shared_fc1"] = None
    gen = torch.Generator().manual_seed(case.seed + 7)
    G = torch.randn(case.T, case.d, generator=gen)
    grad_aux = torch.tensor([g_aux, 0.0, 0.0], device=dev)
    bw = ops.backward_weights(w1b, w2b, sw1b, sw2b)
    g = ops.moe_backward(G.to(bf).to(dev), grad_aux, x, wr_t, bw, state, top_k=case.k,
                         score_fn=case.score_fn, activation=case.activation,
                         aux_coeff=aux_coeff, z_coeff=z_coeff)
    torch.cuda.synchronize()
    ref = reference_grads(cpu["x"], wr, cpu["bias"], cpu["w1"], cpu["w2"], cpu["shared_w1"],
                          cpu["shared_w2"], state["ids"].cpu(), G.to(bf).float(), g_aux, case,
                          aux_coeff, z_coeff)
    names = ["x", "router", "w1", "w2"] + (["shared_w1", "shared_w2"] if sw1b is not None else [])
    for name, r in zip(names, ref):
        got = g[name].float().cpu()
        assert got.shape == r.shape, name
        err = rel_l2(got, r)
        assert err <= TOL, f"{name}: relative L2 {err:.3e}"


@pytest.mark.parametrize("activation", [0, 1])
def test_activation_backward_matches_autograd(activation):
    from nexttransformer_amd import ops
    rows, H = 333, 136
    gen = torch.Generator().manual_seed(5 + activation)
    F = 2 * H if activation == 0 else H
    fc1 = torch.randn(rows, F, generator=gen).to(torch.bfloat16)
    dh = torch.randn(rows, H, generator=gen).to(torch.bfloat16)
    got = ops.act_bwd(fc1.cuda(), dh.cuda(), activation).float().cpu()
    f = fc1.float().requires_grad_()
    if activation == 0:
        h = torch.nn.functional.silu(f[:, :H]) * f[:, H:]
    else:
        h = torch.relu(f).square()
    h.backward(dh.float())
    torch.testing.assert_close(got, f.grad.to(torch.bfloat16).float(), rtol=1.6e-2, atol=1e-5)


def test_combine_backward_is_exact_transpose():
    """grad_y rows are w * grad_out in bf16 and grad_w the fp32 dots (checked in float64)."""
    from nexttransformer_amd import ops
    T, d, E, k = 257, 264, 12, 3
    gen = torch.Generator().manual_seed(9)
    ids = torch.rand(T, E, generator=gen).topk(k, dim=1).indices.int()
    w = torch.rand(T, k, generator=gen)
    counts, offsets, src, perm_w, cdest, cw, _ = ops.route_plan(ids.cuda(), w.cuda(), E, None,
                                                                False)
    y = torch.randn(T * k, d, generator=gen).to(torch.bfloat16)
    g = torch.randn(T, d, generator=gen).to(torch.bfloat16)
    gy, gw = ops.combine_bwd(g.cuda(), y.cuda(), ids.cuda(), cdest, cw)
    torch.cuda.synchronize()
    src_c, pw = src.cpu().long(), perm_w.cpu()
    want = (pw[:, None] * g.float()[src_c]).to(torch.bfloat16)
    assert torch.equal(gy.cpu(), want)
    order = ids.long().argsort(-1)
    dest_topk = torch.empty(T, k, dtype=torch.long)
    dest_topk.scatter_(1, order, cdest.cpu().long())
    ref = (g.double()[:, None, :] * y.double()[dest_topk]).sum(-1)
    torch.testing.assert_close(gw.cpu().double(), ref, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("T,k,shared", [(1, 1, True), (2, 3, False), (37, 8, True),
                                        (515, 4, True), (4099, 8, False)])
def test_combine_row_shapes_agree_bit_for_bit(T, k, shared):
    """The combine walks a row in chunks whose shape depends on d (64-lane chunks, the last
    one partly idle, at d = 256, 1280 and 1344, whole 64-vector chunks at d = 1536, 128-vector
    chunks at d = 2048) but sums every column in the same order, so the first d columns of the
    d = 2048 combine over the same rows equal each narrower one bit for bit; all against
    float64. The shared rows have a row stride other than d."""
    from nexttransformer_amd import ops
    E, D = 16, 2048
    gen = torch.Generator().manual_seed(31 + T + k)
    ids = torch.rand(T, E, generator=gen).topk(k, dim=1).indices.int().cuda()
    w = torch.rand(T, k, generator=gen).cuda()
    counts, _, _, _, cdest, cw, _ = ops.route_plan(ids, w, E, None, False)
    nb = (T + 63) // 64
    pp, zp = torch.rand(nb, E, generator=gen).cuda(), torch.rand(nb, generator=gen).cuda()
    y = torch.randn(T * k, D, generator=gen).to(torch.bfloat16).cuda()
    sh = torch.randn(T, D + 64, generator=gen).to(torch.bfloat16).cuda() if shared else None
    wide, wide_aux = ops.combine_aux(y, cdest, cw, None if sh is None else sh[:, :D], pp, zp,
                                     counts, 0.01, 0.001)
    dest = cdest.cpu().long()
    ref = (cw.cpu().double()[:, :, None] * y.cpu().double()[dest]).sum(1)
    if shared:
        ref += sh[:, :D].cpu().double()
    for d in (256, 1280, 1344, 1536):
        got, aux = ops.combine_aux(y[:, :d].contiguous(), cdest, cw,
                                   None if sh is None else sh[:, :d], pp, zp, counts, 0.01, 0.001)
        assert torch.equal(got, wide[:, :d]), d
        assert torch.equal(aux, wide_aux), d
    torch.testing.assert_close(wide.cpu().double(), ref, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("gather", [False, True])
def test_grouped_wgrad_matches_float64(gather):
    """Ragged segments (empty, shorter than one 32-row step, not a multiple of it, long)."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(31 + gather)
    sizes = [0, 5, 32, 77, 300, 0, 1]
    N, M = 256, 128
    total = sum(sizes)
    offsets = torch.tensor([0] + list(torch.tensor(sizes).cumsum(0)), dtype=torch.int32)
    a = torch.randn(total, N, generator=gen).to(torch.bfloat16)
    b_rows = 50 if gather else total
    b = torch.randn(b_rows, M, generator=gen).to(torch.bfloat16)
    src = torch.randint(0, b_rows, (total,), generator=gen, dtype=torch.int32) if gather else None
    got = ops.grouped_wgrad(a.cuda(), b.cuda(), None if src is None else src.cuda(),
                            offsets.cuda(), total).float().cpu()
    bb = b[src.long()] if gather else b
    for s in range(len(sizes)):
        lo, hi = int(offsets[s]), int(offsets[s + 1])
        ref = a[lo:hi].double().t() @ bb[lo:hi].double()
        if hi == lo:
            assert torch.equal(got[s], torch.zeros(N, M))
        else:
            torch.testing.assert_close(got[s].double(), ref, rtol=8e-3, atol=1e-2)


WGRAD_SHAPES = [(320, 192, False, 1), (192, 320, True, 1), (64, 64, True, 1),
                (320, 1280, True, 1), (1280, 320, False, 1), (128, 256, True, 3),
                (256, 128, False, 4), (256, 256, True, 1), (512, 256, False, 1),
                (256, 768, True, 1), (256, 768, True, 2)]


@pytest.mark.parametrize("N,M,gather,splits", WGRAD_SHAPES,
                         ids=[f"N{n}-M{m}-{'gather' if g else 'rows'}-s{k}"
                              for n, m, g, k in WGRAD_SHAPES])
def test_grouped_wgrad_shapes_fp32_and_bf16(N, M, gather, splits):
    """Every tile shape (256 x 256 when N and M are multiples of 256 and K is not split; else
    N <= M: 128 x 256, else 256 x 128; segments of 1, 2, 3 and 9 slabs against the 256 x 256
    kernel's three-slab copy lead), partial tiles in N and M
    (320 = 256 + 64, 192 = 128 + 64), ragged segments (empty, 1 row, not a multiple of the
    32-row slab, several slabs), gathered B rows (with indices past a slab boundary), split K in
    fixed order; fp32 output against float64 at fp32-accumulation tolerance, bf16 output equal
    to the fp32 result rounded once."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(N + 3 * M + splits)
    sizes = [0, 1, 31, 33, 96, 0, 257, 64]
    total = sum(sizes)
    offsets = torch.tensor([0] + list(torch.tensor(sizes).cumsum(0)), dtype=torch.int32)
    a = torch.randn(total, N, generator=gen).to(torch.bfloat16)
    b_rows = 97 if gather else total
    b = torch.randn(b_rows, M, generator=gen).to(torch.bfloat16)
    src = torch.randint(0, b_rows, (total,), generator=gen, dtype=torch.int32) if gather else None
    args = (a.cuda(), b.cuda(), None if src is None else src.cuda(), offsets.cuda(), total, splits)
    got32 = ops.grouped_wgrad(*args, out_fp32=True).cpu()
    got16 = ops.grouped_wgrad(*args).cpu()
    assert torch.equal(got16, got32.to(torch.bfloat16))
    bb = b[src.long()] if gather else b
    for s in range(len(sizes)):
        lo, hi = int(offsets[s]), int(offsets[s + 1])
        ref = a[lo:hi].double().t() @ bb[lo:hi].double()
        if hi == lo:
            assert torch.equal(got32[s], torch.zeros(N, M))
        else:
            torch.testing.assert_close(got32[s].double(), ref, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("gather,splits", [(False, 1), (True, 1), (True, 2)])
def test_grouped_wgrad_walks_many_tiles(gather, splits):
    """Many tiles (64 segments x 8 tiles of 256 x 256; with split K, two chunks of 16 tiles of
    128 x 256 per segment) over ragged segments: empty segments between non-empty ones, one-row
    and one-slab segments, segments of many slabs; fp32 output against float64."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(7 + 2 * gather + splits)
    S, N, M = 64, 512, 1024
    sizes = torch.randint(0, 160, (S,), generator=gen)
    sizes[torch.randperm(S, generator=gen)[:12]] = 0
    sizes[3], sizes[4], sizes[5], sizes[6] = 1, 32, 33, 300
    total = int(sizes.sum())
    offsets = torch.cat([torch.zeros(1, dtype=torch.int64), sizes.cumsum(0)]).to(torch.int32)
    a = torch.randn(total, N, generator=gen).to(torch.bfloat16)
    b_rows = 211 if gather else total
    b = torch.randn(b_rows, M, generator=gen).to(torch.bfloat16)
    src = torch.randint(0, b_rows, (total,), generator=gen, dtype=torch.int32) if gather else None
    got = ops.grouped_wgrad(a.cuda(), b.cuda(), None if src is None else src.cuda(),
                            offsets.cuda(), total, splits, out_fp32=True).cpu()
    bb = (b[src.long()] if gather else b).double()
    ad = a.double()
    for s in range(S):
        lo, hi = int(offsets[s]), int(offsets[s + 1])
        if hi == lo:
            assert torch.equal(got[s], torch.zeros(N, M)), s
        else:
            torch.testing.assert_close(got[s].double(), ad[lo:hi].t() @ bb[lo:hi], rtol=1e-5,
                                       atol=1e-4, msg=f"segment {s} ({hi - lo} rows)")


# the last two: a partial N tile (ReLU^2, 320 columns: the T3 cell's up projection) and an odd
# K-step count with a six-block N tile (K = 320, SwiGLU 96 columns)
@pytest.mark.parametrize("activation,d,H", [(0, 512, 256), (1, 512, 256), (1, 1280, 320),
                                            (0, 320, 96)],
                         ids=["swiglu", "relu2", "relu2-d1280-H320", "swiglu-d320-H96"])
def test_kept_pre_activations_equal_a_recompute(activation, d, H):
    """The keep launch's h equals the plain packed launch's, and its pre-activations equal an
    EPI_NONE launch over the same rows, bit for bit (same fp32 accumulators, one rounding)."""
    from nexttransformer_amd import _native as nat, ops
    gen = torch.Generator().manual_seed(41 + activation + d)
    E, T = 8, 700
    F = 2 * H if activation == 0 else H
    up = nat.EPI_SWIGLU if activation == 0 else nat.EPI_RELU2
    w1 = (torch.randn(E, F, d, generator=gen) * 0.05).to(torch.bfloat16).cuda()
    x = torch.randn(T, d, generator=gen).to(torch.bfloat16).cuda()
    sizes = torch.tensor([0, 130, 1, 512, 77, 0, 300, 380])
    offsets = torch.cat([torch.zeros(1), sizes.cumsum(0)]).int().cuda()
    A = int(sizes.sum())
    src = torch.randint(0, T, (A,), generator=gen, dtype=torch.int32).cuda()
    h, pre = ops.grouped_gemm_packed_keep(x, src, offsets, ops.pack_expert_weights(w1, up), up, A)
    h_ref = ops.grouped_gemm_packed(x, src, offsets, ops.pack_expert_weights(w1, up), up, A)
    pre_ref = ops.grouped_gemm_packed(x, src, offsets, ops.pack_expert_weights(w1, nat.EPI_NONE),
                                      nat.EPI_NONE, A)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    assert torch.equal(pre, pre_ref)


@pytest.mark.parametrize("activation,K,n_out", [(1, 1280, 320), (1, 320, 320), (0, 1280, 192)],
                         ids=["relu2-K1280-N320", "relu2-K320-N320", "swiglu-K1280-N192"])
def test_kept_pre_activations_plain_weights(activation, K, n_out):
    """Plain-weight keep launch (256 x 256 kernel, the T3 cell's widths): its h equals the plain
    launch's and its pre-activations an EPI_NONE launch over the same rows, bit for bit."""
    from nexttransformer_amd import _native as nat, ops
    gen = torch.Generator().manual_seed(51 + K + activation)
    E, T = 6, 900
    F = 2 * n_out if activation == 0 else n_out
    up = nat.EPI_SWIGLU if activation == 0 else nat.EPI_RELU2
    w1 = (torch.randn(E, F, K, generator=gen) * 0.05).to(torch.bfloat16).cuda()
    x = torch.randn(T, K, generator=gen).to(torch.bfloat16).cuda()
    sizes = torch.tensor([0, 300, 1, 513, 0, 250])
    offsets = torch.cat([torch.zeros(1), sizes.cumsum(0)]).int().cuda()
    A = int(sizes.sum())
    src = torch.randint(0, T, (A,), generator=gen, dtype=torch.int32).cuda()
    assert ops.plain_keep_supported(K, n_out)
    h, pre = ops.grouped_gemm_keep(x, src, offsets, w1, up, A)
    h_ref = ops.grouped_gemm(x, src, offsets, w1, up, A)
    pre_ref = ops.grouped_gemm(x, src, offsets, w1, nat.EPI_NONE, A)
    torch.cuda.synchronize()
    assert pre.shape == (A, F)
    assert torch.equal(h, h_ref)
    assert torch.equal(pre, pre_ref)


def test_convert_expert_weights_is_the_cast_and_its_transpose():
    """One pass over fp32 masters gives exactly torch's round-to-nearest-even bf16 cast and the
    transpose of it, for stacks whose sides are different multiples of 64."""
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(51)
    w = (torch.randn(3, 192, 320, generator=g) * torch.logspace(-6, 2, 320)).cuda()
    out, out_t = ops.convert_expert_weights(w, True, True)
    ref = w.to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(out_t.view(torch.int16), ref.transpose(1, 2).contiguous().view(torch.int16))
    only_t = ops.convert_expert_weights(w, False, True)[1]
    assert torch.equal(only_t, out_t)


@pytest.mark.parametrize("epilogue,R,K", [(0, 192, 320), (1, 320, 256), (2, 128, 384)],
                         ids=["swiglu-R192-K320", "relu2-R320-K256", "plain-R128-K384"])
def test_convert_pack_equals_convert_then_pack(epilogue, R, K):
    """One pass over fp32 masters gives the plain copy, its transpose, the copy packed for the
    epilogue and the transpose packed as a plain projection, equal bit for bit to
    convert_expert_weights followed by pack_expert_weights (SwiGLU with n_out = 96: a 64-row tile
    straddles the gate / value boundary)."""
    from nexttransformer_amd import _native as nat, ops
    g = torch.Generator().manual_seed(61 + epilogue)
    w = torch.randn(3, R, K, generator=g).cuda()
    out, out_t = ops.convert_expert_weights(w, True, True)
    a, at, p, pt = ops.convert_pack_expert_weights(w, epilogue, True, True, True, True)
    ref_p = ops.pack_expert_weights(out, epilogue)
    ref_pt = ops.pack_expert_weights(out_t, nat.EPI_NONE)
    only = ops.convert_pack_expert_weights(w, epilogue, False, False, True, False)
    torch.cuda.synchronize()
    eq = lambda x, y: torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert eq(a, out) and eq(at, out_t) and eq(p, ref_p) and eq(pt, ref_pt) and eq(only[2], ref_p)
    assert only[0].numel() == 0 and only[1].numel() == 0 and only[3].numel() == 0


def test_module_keeps_masters_in_one_buffer_and_falls_back_when_replaced():
    """The experts' fp32 masters are slices of one buffer (the weight cast reads it without a
    stack); an expert whose weight tensor is replaced is still used, through a stacked copy."""
    from nexttransformer_amd.moe import MoELayer
    from nexttransformer_amd.moe_recipe import MoERecipe
    r = MoERecipe(layers=2, width=256, heads=4, routed_experts=8, top_k=2, expert_width=64,
                  activation="swiglu", shared_experts=0, allow_any_expert_width=True,
                  global_batch_tokens=2048)
    m = MoELayer(r, 2)
    w1 = [e.linear_fc1.weight for e in m.experts.local_experts]
    assert all(w.data_ptr() == m._fc1_pool[i].data_ptr() for i, w in enumerate(w1))
    x = torch.randn(300, 256, generator=torch.Generator().manual_seed(52)).to(torch.bfloat16).cuda()
    with torch.no_grad():
        for e in m.experts.local_experts:
            e.linear_fc2.weight.normal_(0, 0.1)
        a, _ = m(x)
        e3 = m.experts.local_experts[3]
        e3.linear_fc1.weight = torch.nn.Parameter(e3.linear_fc1.weight.detach().clone() * 2)
        b, _ = m(x)
        e3.linear_fc1.weight.mul_(0.5)
        c, _ = m(x)
    assert not torch.equal(a, b) and torch.equal(a, c)


def test_module_expert_gradients_accumulate_like_autograd():
    """The routed experts' .grad is set by the layer's backward (they are not autograd inputs):
    taken as fresh slices after zero_grad(set_to_none), accumulated into the same stack when
    every .grad is still its slice, added per tensor when they are mixed, left alone for a
    master that does not require grad; the router's and the shared expert's go through
    autograd. The backward is deterministic, so sums are checked bit for bit."""
    from nexttransformer_amd.moe import MoELayer, set_aux_loss_scale
    from nexttransformer_amd.moe_recipe import MoERecipe
    r = MoERecipe(layers=2, width=256, heads=4, routed_experts=8, top_k=2, expert_width=64,
                  activation="relu2", shared_experts=1, shared_expert_width=64,
                  allow_any_expert_width=True, global_batch_tokens=2048)
    m = MoELayer(r, 2)
    set_aux_loss_scale(1.0, device="cuda")
    gen = torch.Generator().manual_seed(61)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.05)
    x = torch.randn(300, 256, generator=gen).to(torch.bfloat16).cuda()
    G = torch.randn(300, 256, generator=gen).to(torch.bfloat16).cuda()
    params = dict(m.named_parameters())
    experts = [n for n in params if ".local_experts." in n]
    assert len(experts) == 16

    def backward():
        out, _ = m(x)
        out.backward(G)

    m.zero_grad(set_to_none=True)
    backward()
    once = {n: p.grad.clone() for n, p in params.items()}
    assert all(torch.isfinite(g).all() and g.abs().sum() > 0 for g in once.values())
    ptr0 = params[experts[0]].grad.data_ptr()
    backward()  # accumulate: every expert .grad is still its slice of the stack
    for n, p in params.items():
        assert torch.equal(p.grad, 2 * once[n]), n
    assert params[experts[0]].grad.data_ptr() == ptr0
    m.zero_grad(set_to_none=False)
    backward()
    for n, p in params.items():
        assert torch.equal(p.grad, once[n]), n
    # mixed: one expert's .grad cleared, one replaced by a tensor of its own
    params[experts[3]].grad = None
    params[experts[5]].grad = torch.ones_like(once[experts[5]])
    backward()
    for n, p in params.items():
        want = once[n] if n == experts[3] else (
            1 + once[n] if n == experts[5] else 2 * once[n])
        assert torch.equal(p.grad, want), n
    # a frozen expert master keeps no gradient
    m.zero_grad(set_to_none=True)
    params[experts[6]].requires_grad_(False)
    backward()
    assert params[experts[6]].grad is None
    assert torch.equal(params[experts[7]].grad, once[experts[7]])


@pytest.mark.parametrize("E,Fs", [(40, 64), (256, 320), (8, 0), (37, 16)])
def test_backward_first_operand_is_the_split_and_concatenation(E, Fs):
    """[dfc1s | g_hi | g_hi | g_lo | 0] bit for bit against split_bf16 and torch slicing: E not a
    multiple of the 32-wide blocks (nor of 8: element-wise loads instead of vector loads), values
    spanning exponents, exact bf16 values (lo = 0), negative zero, no shared expert."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(E + Fs)
    T = 333
    Ep = (E + 31) // 32 * 32
    Kc = (Fs + 3 * Ep + 63) // 64 * 64
    g = torch.randn(T, E, generator=gen) * torch.exp2(torch.randint(-30, 30, (T, E),
                                                                   generator=gen).float())
    g[0] = g[0].to(torch.bfloat16).float()
    g[1, :4] = torch.tensor([0.0, -0.0, 1.0, -3.5])
    dfc1s = torch.randn(T, Fs, generator=gen).to(torch.bfloat16) if Fs else None
    got = ops.backward_first_operand(g.cuda(), None if dfc1s is None else dfc1s.cuda(), Ep,
                                     Kc).cpu()
    hi, lo = ops.split_bf16(g)
    want = torch.zeros(T, Kc, dtype=torch.bfloat16)
    if Fs:
        want[:, :Fs] = dfc1s
    want[:, Fs:Fs + E] = hi
    want[:, Fs + Ep:Fs + Ep + E] = hi
    want[:, Fs + 2 * Ep:Fs + 2 * Ep + E] = lo
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("E,d,dp,Fs", [(32, 1024, 1024, 0), (8, 40, 64, 0),
                                       (256, 1280, 1280, 640), (40, 96, 128, 192)])
def test_router_operands_match_the_torch_construction(E, d, dp, Fs):
    """router_operands' w_router_t and first operand, bit for bit against torch: the zero-padded
    transpose, and [S^T | hi | lo | hi | 0] from split_bf16 (E not a multiple of 32, d padded to
    dp, values spanning exponents, exact bf16 values, negative zero, with and without a shared
    expert); without want_first only w_router_t."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(E + d + Fs)
    w = torch.randn(E, d, generator=gen) * torch.exp2(
        torch.randint(-30, 30, (E, d), generator=gen).float())
    w[0] = w[0].to(torch.bfloat16).float()
    w[1, :4] = torch.tensor([0.0, -0.0, 1.0, -3.5])
    s = (torch.randn(Fs, dp, generator=gen).to(torch.bfloat16) if Fs else None)
    rt, first = ops.router_operands(w.cuda(), dp, None if s is None else s.cuda(), True)
    want_rt = torch.zeros(dp, E)
    want_rt[:d] = w.t()
    assert torch.equal(rt.cpu().view(torch.int32), want_rt.view(torch.int32))
    Ep, Kc = ops.first_layout(E, Fs)
    hi, lo = ops.split_bf16(want_rt)
    want = torch.zeros(1, dp, Kc, dtype=torch.bfloat16)
    if Fs:
        want[0, :, :Fs] = s.t()
    want[0, :, Fs:Fs + E] = hi
    want[0, :, Fs + Ep:Fs + Ep + E] = lo
    want[0, :, Fs + 2 * Ep:Fs + 2 * Ep + E] = hi
    assert first.shape == (1, dp, Kc)
    assert torch.equal(first.cpu().view(torch.int16), want.view(torch.int16))
    rt2, none = ops.router_operands(w.cuda(), dp, None, False)
    assert none.numel() == 0 and torch.equal(rt2.cpu().view(torch.int32), want_rt.view(torch.int32))


@pytest.mark.parametrize("N0,M0,N1,M1", [(512, 256, 256, 512), (256, 256, 320, 256)],
                         ids=["one-launch", "two-launches"])
def test_grouped_wgrad_pair_equals_two_calls(N0, M0, N1, M1):
    """grouped_wgrad_pair bit for bit against two grouped_wgrad calls (fp32 and bf16 output) over
    ragged segments (empty, one row, partial slabs, many slabs), the first product gathered: as
    one launch of the 256 x 256 kernel over both tile lists, and (a width not a multiple of 256)
    as two launches; and against float64."""
    from nexttransformer_amd import ops
    gen = torch.Generator().manual_seed(N0 + M1)
    sizes = [0, 1, 33, 96, 0, 257, 64, 700]
    total = sum(sizes)
    offsets = torch.tensor([0] + list(torch.tensor(sizes).cumsum(0)), dtype=torch.int32).cuda()
    b_rows = 131
    a0 = torch.randn(total, N0, generator=gen).to(torch.bfloat16).cuda()
    b0 = torch.randn(b_rows, M0, generator=gen).to(torch.bfloat16).cuda()
    src = torch.randint(0, b_rows, (total,), generator=gen, dtype=torch.int32).cuda()
    a1 = torch.randn(total, N1, generator=gen).to(torch.bfloat16).cuda()
    b1 = torch.randn(total, M1, generator=gen).to(torch.bfloat16).cuda()
    for f32 in (True, False):
        c0, c1 = ops.grouped_wgrad_pair(a0, b0, src, a1, b1, None, offsets, total, f32)
        w0 = ops.grouped_wgrad(a0, b0, src, offsets, total, 1, f32)
        w1 = ops.grouped_wgrad(a1, b1, None, offsets, total, 1, f32)
        assert torch.equal(c0, w0) and torch.equal(c1, w1)
    bb0 = b0[src.long()].double().cpu()
    for s in range(len(sizes)):
        lo, hi = int(offsets[s]), int(offsets[s + 1])
        ref0 = a0[lo:hi].double().cpu().t() @ bb0[lo:hi]
        ref1 = a1[lo:hi].double().cpu().t() @ b1[lo:hi].double().cpu()
        torch.testing.assert_close(c0[s].double().cpu(), ref0.to(torch.bfloat16).double(),
                                   rtol=1e-2, atol=1e-2)
        torch.testing.assert_close(c1[s].double().cpu(), ref1.to(torch.bfloat16).double(),
                                   rtol=1e-2, atol=1e-2)
