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
