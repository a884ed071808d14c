"""GPU checks of the drop-in boundary: the committed golden vectors through the ntmoe ops, the MoE
module (reference constructor, parameter contract, (out, aux_loss) forward, last_load) and the
ffn plugin, against the CPU oracle.

Bar: routing bit-exact; outputs within relative L2 1e-2 of the fp32 reference computed from the
same bf16 inputs and bf16-rounded weights; aux within 1e-5 relative.
Reference anchors: megatron_moe.py:124-182; tests/test_megatron_moe.py:126-166.
"""
from types import SimpleNamespace

import pytest
import torch

from oracle import moe_oracle as orc
from tests.moe_cases import rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
AUX_RTOL = 1e-5


def test_golden_vectors_through_ops():
    from nexttransformer_amd import ops
    from tests.golden_io import load_golden
    dev = torch.device("cuda")
    for name, c in load_golden().items():
        print(f"[golden] {name}: T={c['T']} d={c['d']} E={c['E']} k={c['k']}", flush=True)
        sw1 = None if c["shared_w1"] is None else c["shared_w1"][None].to(dev)
        sw2 = None if c["shared_w2"] is None else c["shared_w2"][None].to(dev)
        out, aux, st = ops.moe_forward(
            c["x"].to(dev), c["router"].t().contiguous().to(dev), c["w1"].to(dev),
            c["w2"].to(dev), top_k=c["k"], score_fn=c["score_fn"], activation=c["activation"],
            logit_bias=None if c["bias"] is None else c["bias"].to(dev), shared_w1=sw1,
            shared_w2=sw2, want_logits=True)
        torch.cuda.synchronize()
        assert torch.equal(st["logits"].cpu().view(torch.int32), c["ref_logits"].view(torch.int32)), name
        assert torch.equal(st["ids"].cpu(), c["ref_ids"]), name
        # routing weights are floating point: the fp32 kernel against the oracle's double
        torch.testing.assert_close(st["weights"].cpu(), c["ref_weights"], rtol=2e-6, atol=2e-7)
        assert torch.equal(st["counts"].cpu(), c["ref_counts"]), name
        assert torch.equal(st["offsets"].cpu(), c["ref_offsets"]), name
        assert torch.equal(st["src_row"].cpu(), c["ref_src_row"]), name
        # the combine plan lists each token's rows in ascending expert order (the order the
        # combine kernel sums them in); the oracle's dest is in top-k slot order
        by_expert = c["ref_ids"].long().argsort(dim=1)
        assert torch.equal(st["combine_dest"].cpu(), c["ref_dest"].gather(1, by_expert)), name
        assert rel_l2(out.float(), c["ref_out"]) <= BF16_TOL, name
        for got, want in zip(aux.cpu().tolist(), c["ref_aux"].tolist()):
            assert got == pytest.approx(want, rel=AUX_RTOL, abs=1e-9), name


def _recipe(**kw):
    from nexttransformer_amd.moe_recipe import MoERecipe
    base = dict(layers=4, width=256, heads=4, routed_experts=8, top_k=2, expert_width=64,
                global_batch_tokens=2048)
    base.update(kw)
    return MoERecipe(**base)


def _randomise_fc2(m, seed):
    """fc2 starts at zero (megatron_moe.py:112); nonzero weights avoid a vacuous check."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        experts = list(m.experts.local_experts)
        if m.shared_experts is not None:
            experts.append(m.shared_experts)
        for e in experts:
            w = e.linear_fc2.weight
            w.copy_((torch.randn(w.shape, generator=g) * 0.1).to(w.device))


def _oracle_for(m, hidden):
    r = m.recipe
    bf = lambda t: t.detach().cpu().to(torch.bfloat16).float()
    experts = m.experts.local_experts
    w = orc.Weights(router=m.router.weight.detach().cpu(),
                    w1=torch.stack([bf(e.linear_fc1.weight) for e in experts]),
                    w2=torch.stack([bf(e.linear_fc2.weight) for e in experts]),
                    shared_w1=None if m.shared_experts is None else bf(m.shared_experts.linear_fc1.weight),
                    shared_w2=None if m.shared_experts is None else bf(m.shared_experts.linear_fc2.weight))
    return orc.moe_forward(hidden.reshape(-1, r.width).cpu().to(torch.bfloat16), w, r.top_k,
                           score_fn=orc.SIGMOID if r.score_function == "sigmoid" else orc.SOFTMAX,
                           activation=orc.SWIGLU if r.activation == "swiglu" else orc.RELU2,
                           aux_coeff=r.aux_loss_coeff, z_coeff=r.z_loss_coeff)


@pytest.mark.parametrize("kw", [
    dict(),                                                        # reference recipe: ReLU^2 + shared
    dict(activation="swiglu", shared_experts=0, expert_width=128, allow_any_expert_width=True),
    dict(score_function="sigmoid", routed_experts=32, top_k=8, activation="swiglu",
         shared_expert_width=192, allow_any_expert_width=True),
    dict(width=32, heads=2, expert_width=8),                       # the reference debug shape, padded
], ids=["relu2-shared", "swiglu", "sigmoid-shared", "debug-width-32"])
def test_module_forward_matches_oracle(kw):
    from nexttransformer_amd.moe import MoELayer
    r = _recipe(**kw)
    m = MoELayer(r, 2)
    _randomise_fc2(m, 1)
    g = torch.Generator().manual_seed(2)
    hidden = torch.randn(3, 70, r.width, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        out, aux = m(hidden)
    torch.cuda.synchronize()
    ref = _oracle_for(m, hidden)
    assert out.shape == hidden.shape and out.dtype == torch.bfloat16
    assert rel_l2(out.float().reshape(-1, r.width), ref["out"]) <= BF16_TOL
    assert torch.equal(m.last_load.cpu(), ref["counts"].long())
    assert m.last_load.dtype == torch.int64 and int(m.last_load.sum()) == 210 * r.top_k
    assert aux.dim() == 0 and m.last_aux_loss is aux
    assert aux.item() == pytest.approx(ref["aux"], rel=AUX_RTOL)


def test_module_forward_at_t3_expert_cell_shape():
    """The reference's registered recipe cell moe-T3-L20 (width 1280, 256 experts, top-8, ReLU^2
    experts of width 320, one shared expert of width 320; megatron_moe.py:23-24,41,51), one
    layer on 200 tokens, against the oracle."""
    from pathlib import Path
    from nexttransformer_amd.moe import MoELayer
    from nexttransformer_amd.moe_recipe import load_t3_recipe
    root = Path(__file__).resolve().parents[1]
    r = load_t3_recipe("moe-T3-L20", root / "tests" / "golden" / "t3_expert_cells.json")
    assert (r.width, r.routed_experts, r.top_k, r.expert_width, r.activation) == \
        (1280, 256, 8, 320, "relu2")
    m = MoELayer(r, 2)
    _randomise_fc2(m, 3)
    g = torch.Generator().manual_seed(4)
    hidden = torch.randn(2, 100, r.width, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        out, aux = m(hidden)
    torch.cuda.synchronize()
    ref = _oracle_for(m, hidden)
    assert rel_l2(out.float().reshape(-1, r.width), ref["out"]) <= BF16_TOL
    assert torch.equal(m.last_load.cpu(), ref["counts"].long())
    assert aux.item() == pytest.approx(ref["aux"], rel=AUX_RTOL)


@pytest.mark.parametrize("kw", [
    dict(activation="swiglu", width=512, heads=4, expert_width=256, allow_any_expert_width=True),
    dict(width=96, heads=2, expert_width=24),  # ReLU^2 + shared, padded to 128
], ids=["swiglu-512", "relu2-shared-padded"])
def test_module_fp8_matches_dequantised_reference(kw):
    """The module quantises its fp32 masters (zero-padded to multiples of 128) per 128 x 128 block
    and packs them; the reference quantises the same padded masters with the oracle."""
    from nexttransformer_amd.moe import MoELayer
    r = _recipe(expert_dtype="fp8", **kw)
    m = MoELayer(r, 2)
    _randomise_fc2(m, 6)
    hidden = torch.randn(2, 40, r.width).to(torch.bfloat16).cuda()
    with torch.no_grad():
        out, aux = m(hidden)
    p = m.packed_weights()
    assert p["w1"].dtype == torch.uint8 and p["packed"]
    gated = r.activation == "swiglu"
    act = orc.SWIGLU if gated else orc.RELU2
    dp = p["router_t"].shape[0]
    up128 = lambda n: (n + 127) // 128 * 128

    def padded(experts, hidden_w):
        hp = up128(hidden_w)
        n = len(experts)
        w1 = torch.zeros(n, (2 if gated else 1) * hp, dp)
        w2 = torch.zeros(n, dp, hp)
        for i, e in enumerate(experts):
            fc1 = e.linear_fc1.weight.detach().cpu()
            if gated:
                w1[i, :hidden_w, :r.width] = fc1[:hidden_w]
                w1[i, hp:hp + hidden_w, :r.width] = fc1[hidden_w:]
            else:
                w1[i, :hidden_w, :r.width] = fc1
            w2[i, :r.width, :hidden_w] = e.linear_fc2.weight.detach().cpu()
        return orc.quantize_blockwise(w1) + orc.quantize_blockwise(w2)

    w1q, w1s, w2q, w2s = padded(list(m.experts.local_experts), r.expert_width)
    assert torch.equal(w1s, p["w1_scale"].cpu()) and torch.equal(w2s, p["w2_scale"].cpu())
    shared = None
    if m.shared_experts is not None:
        sq = padded([m.shared_experts], r.shared_expert_width)
        shared = tuple(t[0] for t in sq)
    x = torch.nn.functional.pad(hidden.reshape(-1, r.width).cpu(), (0, dp - r.width))
    ref = orc.moe_forward_fp8(x, torch.nn.functional.pad(m.router.weight.detach().cpu(),
                                                         (0, dp - r.width)),
                              w1q, w1s, w2q, w2s, r.top_k, activation=act, shared=shared)
    ref_out = ref["out"][:, :r.width]
    assert torch.equal(m.last_load.cpu(), ref["counts"].long())
    assert rel_l2(out.float().reshape(-1, r.width), ref_out) <= 3e-2


def test_module_empty_experts_256_top8():
    """tests/test_megatron_moe.py:157-166: two tokens over 256 experts."""
    from nexttransformer_amd.moe import MoELayer
    m = MoELayer(_recipe(routed_experts=256, top_k=8), 2)
    _randomise_fc2(m, 3)
    hidden = torch.randn(1, 2, 256).to(torch.bfloat16).cuda()
    with torch.no_grad():
        out, _ = m(hidden)
    ref = _oracle_for(m, hidden)
    assert int(m.last_load.sum()) == 16 and int((m.last_load == 0).sum()) > 0
    assert rel_l2(out.float().reshape(-1, 256), ref["out"]) <= BF16_TOL


def test_module_repacks_after_in_place_update_and_casts_inputs():
    from nexttransformer_amd.moe import MoEFFN
    ffn = MoEFFN(_recipe(activation="swiglu", expert_width=64), 3)
    m = ffn.engine
    _randomise_fc2(m, 4)
    hidden = torch.randn(2, 16, 256).cuda()
    with torch.no_grad():
        a = ffn(hidden)
        assert a.dtype == torch.float32 and ffn.engine.last_aux_loss is not None
        b = ffn(hidden.to(torch.bfloat16))
        assert torch.equal(a.to(torch.bfloat16), b)
        for e in m.experts.local_experts:
            e.linear_fc2.weight.mul_(2.0)
        m.shared_experts.linear_fc2.weight.mul_(2.0)
        c = ffn(hidden.to(torch.bfloat16))
    assert rel_l2(c.float(), 2 * b.float()) <= 1e-2
    # gradients enabled: the training path gives the same output and fills every .grad
    d = ffn(hidden.to(torch.bfloat16))
    assert torch.equal(d, c)
    d.float().square().sum().backward()  # the engine injects the aux-loss gradient itself
    for name, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name


def test_module_empty_batch():
    from nexttransformer_amd.moe import MoELayer
    m = MoELayer(_recipe(), 2)
    with torch.no_grad():
        out, aux = m(torch.empty(0, 5, 256, dtype=torch.bfloat16, device="cuda"))
    assert out.shape == (0, 5, 256) and aux.item() == 0.0
    assert int(m.last_load.sum()) == 0


def test_plugin_ffn_forward():
    import json
    from pathlib import Path
    from nexttransformer_amd.plugins import nt_moe
    spec = json.loads((Path(nt_moe.__file__).parent / "method.json").read_text())
    opts = dict(spec["options"], routed_experts=16, top_k=4)
    config = SimpleNamespace(method="nt_moe", width=128, heads=4, layers=4, sequence_len=32,
                             vocab_size=128, mlp_width=512, option=lambda n: opts[n])
    module = nt_moe.ffn(config, 1)
    _randomise_fc2(module.engine, 5)
    x = torch.randn(2, 32, 128).to(torch.bfloat16).cuda()
    with torch.no_grad():
        y = module(x)
    ref = _oracle_for(module.engine, x)
    assert y.shape == x.shape and torch.is_tensor(module.last_aux)
    assert rel_l2(y.float().reshape(-1, 128), ref["out"]) <= BF16_TOL
