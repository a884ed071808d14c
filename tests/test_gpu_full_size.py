"""Parity at the benchmark configurations' full sizes (configs 2-4 and the T3 cell, bf16), where
the CPU oracle cannot run the whole layer in seconds: routing and outputs are checked bit-exact / within the
bf16 tolerance on a sample of tokens (each token's output depends only on its own row and its
routing), and the whole-batch results through size-independent properties -- counts sum to
T k and match the ids, the permutation is expert-major and token-ascending with every token
k times, the aux losses equal their closed forms on the kernel's own (bit-checked) logits, and
two runs are bit-identical.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.moe_cases import CONFIGS, make_inputs, rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _run(case, packed):
    from nexttransformer_amd import _native as nat
    from nexttransformer_amd import ops
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2

    pk_up, pk_down = (packed, packed) if isinstance(packed, bool) else packed

    def bf(t, epi, pk):
        if t is None:
            return None
        t = t.to(torch.bfloat16).to(dev)
        return ops.pack_expert_weights(t, epi) if pk else t
    g = dict(x=cpu["x"].to(dev), wt=cpu["router"].t().contiguous().to(dev),
             w1=bf(cpu["w1"], up, pk_up), w2=bf(cpu["w2"], nat.EPI_NONE, pk_down),
             sw1=bf(cpu["shared_w1"], up, pk_up), sw2=bf(cpu["shared_w2"], nat.EPI_NONE, pk_down),
             bias=None if cpu["bias"] is None else cpu["bias"].to(dev))

    def fwd():
        return ops.moe_forward(g["x"], g["wt"], g["w1"], g["w2"], top_k=case.k,
                               score_fn=case.score_fn, activation=case.activation,
                               logit_bias=g["bias"], shared_w1=g["sw1"], shared_w2=g["sw2"],
                               want_logits=True, packed=packed)
    return cpu, fwd


# config 6 (the registered T3 cell: d=1280 is 10 router chunks; K=320 has no packed-weight
# form) runs on plain weights, and with the up projections packed (the module's choice there)
FULL = [(c, p) for c in (2, 3, 4) for p in (False, True)] + [(6, False), (6, (True, False))]


@pytest.mark.parametrize("cfg,packed", FULL, ids=[
    f"{c}-" + ({False: "plain", True: "packed"}[p] if isinstance(p, bool) else "packed-up")
    for c, p in FULL])
def test_full_size_layer(cfg, packed):
    case = CONFIGS[cfg]
    print(f"[full-size] config {cfg} packed={packed}: {case}", flush=True)
    cpu, fwd = _run(case, packed)
    out, aux, st = fwd()
    torch.cuda.synchronize()
    T, E, k = case.T, case.E, case.k
    ids = st["ids"].cpu()
    counts = st["counts"].cpu().long()
    offsets = st["offsets"].cpu().long()
    src = st["src_row"].cpu().long()
    logits = st["logits"].cpu()

    # whole batch: counts, offsets and the permutation
    assert int(counts.sum()) == T * k
    assert torch.equal(counts, torch.bincount(ids.flatten().long(), minlength=E))
    assert offsets[0] == 0 and torch.equal(offsets[1:], counts.cumsum(0))
    assert torch.equal(torch.bincount(src, minlength=T), torch.full((T,), k))
    expert_of_row = torch.repeat_interleave(torch.arange(E), counts)
    key = expert_of_row * T + src  # expert-major, token-ascending <=> strictly increasing
    assert bool((key[1:] > key[:-1]).all())
    rows_of = ids.long()[src]  # the expert each permuted row's token chose, among its k
    assert bool((rows_of == expert_of_row[:, None]).any(1).all())
    # whole batch: the kernel routes every token as top-k of the reference's own router
    # expression F.linear(x.float(), W.float()) (+ bias) does (megatron_moe.py:95-99)
    ref_ids_all, _ = orc.topk(orc.router_logits_reference(cpu["x"], cpu["router"], cpu["bias"]),
                              k, case.score_fn)
    assert torch.equal(ids, ref_ids_all)

    # sampled tokens: fixed-order logits, top-k and outputs against the oracle
    rng = np.random.default_rng(cfg)
    tokens = torch.as_tensor(np.sort(rng.choice(T, 256, replace=False)))
    ref_logits = orc.router_logits_fixed(cpu["x"][tokens], cpu["router"], cpu["bias"])
    assert torch.equal(logits[tokens].view(torch.int32), ref_logits.view(torch.int32))
    ref_ids, _ = orc.topk(ref_logits, k, case.score_fn)
    assert torch.equal(ids[tokens], ref_ids)
    r = lambda t: None if t is None else t.to(torch.bfloat16).float()
    weights = orc.Weights(router=cpu["router"], w1=r(cpu["w1"]), w2=r(cpu["w2"]),
                          shared_w1=None if cpu["shared_w1"] is None else r(cpu["shared_w1"])[0],
                          shared_w2=None if cpu["shared_w2"] is None else r(cpu["shared_w2"])[0],
                          bias=cpu["bias"])
    ref_out = orc.moe_forward_tokens(cpu["x"], weights, k, tokens, logits=logits,
                                     score_fn=case.score_fn, activation=case.activation)
    assert rel_l2(out.cpu()[tokens].float(), ref_out) <= BF16_TOL

    # aux on the kernel's logits (bit-checked above on the sample) in closed form
    lb, z = orc.aux_losses(logits, counts, k, 0.01, 0.001, case.score_fn)
    assert aux[1].item() == pytest.approx(lb, rel=1e-4)
    assert aux[2].item() == pytest.approx(z, rel=1e-4)

    # determinism
    out2, aux2, st2 = fwd()
    assert torch.equal(out2.view(torch.int16), out.view(torch.int16))
    assert torch.equal(aux2, aux) and torch.equal(st2["src_row"], st["src_row"])
    if case.zipf_bias:
        print(f"[full-size] load max/mean {counts.max().item() / counts.float().mean().item():.2f}")


def _layer_from_case(case, cpu):
    """An MoELayer (aux gradient through the returned loss) holding the case's weights as its
    fp32 masters: the module's own training path (fused conversion, packed operands and packed
    transposes where the widths allow, split-K weight gradients at full size)."""
    from nexttransformer_amd.moe import MoELayer
    from nexttransformer_amd.moe_recipe import MoERecipe
    r = MoERecipe(layers=2, width=case.d, heads=max(1, case.d // 64), sequence_len=case.T,
                  global_batch_tokens=case.T, routed_experts=case.E, top_k=case.k,
                  expert_width=case.H, score_function=("softmax", "sigmoid")[case.score_fn],
                  activation=("swiglu", "relu2")[case.activation],
                  shared_experts=1 if case.shared_H else 0,
                  shared_expert_width=case.shared_H or None, allow_any_expert_width=True)
    m = MoELayer(r, 1, aux_grad="loss")
    with torch.no_grad():
        m.router.weight.copy_(cpu["router"])
        for i, e in enumerate(m.experts.local_experts):
            e.linear_fc1.weight.copy_(cpu["w1"][i])
            e.linear_fc2.weight.copy_(cpu["w2"][i])
        if case.shared_H:
            m.shared_experts.linear_fc1.weight.copy_(cpu["shared_w1"][0])
            m.shared_experts.linear_fc2.weight.copy_(cpu["shared_w2"][0])
    return m


@pytest.mark.parametrize("cfg", [2, 6], ids=["config2", "t3-cell"])
def test_full_size_backward_matches_fp32_autograd(cfg):
    """Training step of the module at full size (config 2: T 16384, d 1024, 32 experts, top-4,
    SwiGLU 512; the T3 cell: d 1280, 256 experts, top-8, ReLU^2 320 plus a shared expert):
    every gradient (hidden, router, each expert's fc1 and fc2, the shared expert's) against
    fp32 autograd of the layer written in plain PyTorch on the CPU with the same selection
    (tests/test_megatron_moe.py:126-141 is the reference's small-size analogue), relative L2
    <= 2e-2 per tensor; and a second step's gradients equal the first's bit for bit."""
    case = CONFIGS[cfg]
    cpu = make_inputs(case)
    m = _layer_from_case(case, cpu)
    gen = torch.Generator().manual_seed(case.seed + 11)
    G = torch.randn(case.T, case.d, generator=gen).to(torch.bfloat16)
    g_aux, Gd = 2.0, G.cuda()
    hidden = cpu["x"].cuda()

    def step():
        m.zero_grad(set_to_none=True)
        h = hidden.clone().requires_grad_()
        out, aux = m(h)
        ((out.float() * Gd.float()).sum() + g_aux * aux).backward()
        torch.cuda.synchronize()
        return [h.grad.clone()] + [p.grad.clone() for p in m.parameters()]

    first = step()
    again = step()
    for a, b in zip(first, again):
        assert torch.equal(a, b)
    experts = list(m.experts.local_experts)
    sw = m.shared_experts
    ref = _reference_grads_full(cpu["x"], cpu["router"], cpu["w1"], cpu["w2"], cpu["shared_w1"],
                                cpu["shared_w2"], _selection(m, hidden), G.float(), g_aux, case,
                                m.recipe.aux_loss_coeff, m.recipe.z_loss_coeff)
    x_ref, router_ref, w1_ref, w2_ref = ref[:4]
    assert rel_l2(first[0].float().cpu(), x_ref) <= 2e-2
    assert rel_l2(m.router.weight.grad.cpu(), router_ref) <= 2e-2
    w1_got = torch.stack([e.linear_fc1.weight.grad for e in experts]).cpu()
    w2_got = torch.stack([e.linear_fc2.weight.grad for e in experts]).cpu()
    assert rel_l2(w1_got, w1_ref) <= 2e-2
    assert rel_l2(w2_got, w2_ref) <= 2e-2
    # per expert too (an expert that received no tokens has zero gradients on both sides)
    for i in range(case.E):
        if w1_ref[i].norm() > 0:
            assert rel_l2(w1_got[i], w1_ref[i]) <= 2e-2, i
            assert rel_l2(w2_got[i], w2_ref[i]) <= 2e-2, i
    if sw is not None:
        assert rel_l2(sw.linear_fc1.weight.grad.cpu(), ref[4][0]) <= 2e-2
        assert rel_l2(sw.linear_fc2.weight.grad.cpu(), ref[5][0]) <= 2e-2


def _selection(m, hidden):
    """The experts the layer selected for each token (its route plan is not exposed by the
    module), read back from the forward's ids through a no-grad call of the ops."""
    from nexttransformer_amd import ops
    w = m.packed_weights()
    _, ids, _, _, _ = ops.router(hidden, w["router_t"], m.logit_bias, m.recipe.top_k,
                                 0 if m.recipe.score_function == "softmax" else 1, False)
    return ids.cpu()


def _reference_grads_full(x, wr, w1, w2, sw1, sw2, ids, G, g_aux, case, aux_coeff, z_coeff):
    """fp32 autograd of the layer on the CPU for loss = <out, G> + g_aux (lb + z), with the
    given selection: the same formulas as tests/test_gpu_backward.reference_grads, the expert
    outputs gathered into one index_add so the graph holds each assignment's rows once."""
    from tests.test_gpu_backward import ffn
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
    ids = ids.long()
    sel = logits.gather(1, ids)
    if case.score_fn == 0:
        w = sel.softmax(-1)
    else:
        s = torch.sigmoid(sel)
        w = s / s.sum(-1, keepdim=True)
    toks, rows = [], []
    for e in range(E):
        tok, slot = torch.where(ids == e)
        if tok.numel():
            toks.append(tok)
            rows.append(ffn(x[tok], w1[e], w2[e], case.activation) * w[tok, slot, None])
    out = torch.zeros(T, x.shape[1]).index_add(0, torch.cat(toks), torch.cat(rows))
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
    ((out * G).sum() + g_aux * (lb + z)).backward()
    return [t.grad for t in params]
