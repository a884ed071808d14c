"""GPU checks of the drop-in's training semantics: the aux / z-loss gradient on its own, MCore's
aux-loss autoscaler (megatron_moe.py:233-236; tests/test_megatron_moe.py:183-197), the plugin
shell's loss route counting the aux loss once (lm.py:386-388), the scaling adapter built from a
reference-shaped recipe (megatron_moe.py:185-208), and the module's gradients against fp32
autograd.
"""
from types import SimpleNamespace

import pytest
import torch

from oracle import moe_oracle as orc
from tests.moe_cases import Case, make_inputs, rel_l2
from tests.test_gpu_backward import reference_grads
from tests.test_gpu_module import _oracle_for, _randomise_fc2

pytestmark = pytest.mark.gpu


def _aux_reference(logits, counts, k, score_fn, aux_coeff, z_coeff, g_lb, g_z):
    """d(g_lb * lb + g_z * z)/d logits in float64 on the CPU (the closed forms)."""
    L = logits.detach().cpu().double().requires_grad_()
    T, E = L.shape
    if score_fn == 0:
        p = L.softmax(-1)
    else:
        s = torch.sigmoid(L)
        p = s / s.sum(-1, keepdim=True)
    lb = aux_coeff * E / (k * T * T) * (p.sum(0) * counts.double().cpu()).sum()
    z = z_coeff * torch.logsumexp(L, -1).square().mean()
    (g_lb * lb + g_z * z).backward()
    return L.grad


@pytest.mark.parametrize("E,k,score_fn", [(40, 3, 0), (40, 3, 1), (200, 8, 0), (200, 8, 1)],
                         ids=["E40-softmax", "E40-sigmoid", "E200-softmax", "E200-sigmoid"])
def test_aux_gradient_terms_alone(E, k, score_fn):
    """The router backward with a zero routing-weight gradient: only the load-balance and z-loss
    terms remain, checked one aux output at a time ({lb + z, lb, z} gradients (1,0,0), (0,1,0),
    (0,0,1)) against float64 autograd, with coefficients large enough that a wrong sign or
    scale in either term shows; E is not a multiple of the 64-lane wave."""
    from nexttransformer_amd import ops
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(31 + E + score_fn)
    T, d = 333, 128
    x = torch.randn(T, d, generator=g).to(torch.bfloat16).to(dev)
    wr_t = (torch.randn(E, d, generator=g) * 0.2).t().contiguous().to(dev)
    logits, ids, w, _, _ = ops.router(x, wr_t, None, k, score_fn, True)
    counts = torch.bincount(ids.flatten().long(), minlength=E).to(torch.int32)
    aux_coeff, z_coeff = 1.0, 0.5
    zero = torch.zeros_like(w)
    for ga in ([1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0]):
        got = ops.router_bwd(logits, ids, w, zero, counts, score_fn,
                             torch.tensor(ga, device=dev), aux_coeff, z_coeff).double().cpu()
        ref = _aux_reference(logits, counts, k, score_fn, aux_coeff, z_coeff,
                             ga[0] + ga[1], ga[0] + ga[2])
        assert ref.norm() > 0
        assert rel_l2(got, ref) <= 1e-5, (ga, rel_l2(got, ref))
        torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-6 * ref.abs().max().item())


@pytest.mark.parametrize("score_fn", [0, 1], ids=["softmax", "sigmoid"])
def test_aux_only_layer_gradients(score_fn):
    """moe_backward with a zero output gradient: the router weight and input gradients are
    those of the aux losses alone (dlogits^T x and dlogits Wr), against fp32 autograd."""
    from nexttransformer_amd import ops
    case = Case("aux-only", 300, 256, 40, 4, 128, score_fn=score_fn, seed=33)
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    bf = torch.bfloat16
    x = cpu["x"].to(dev)
    wr_t = cpu["router"].t().contiguous().to(dev)
    w1b, w2b = cpu["w1"].to(bf).to(dev), cpu["w2"].to(bf).to(dev)
    aux_coeff, z_coeff = 1.0, 0.5
    out, aux, state = ops.moe_forward(x, wr_t, w1b, w2b, top_k=case.k, score_fn=score_fn,
                                      aux_coeff=aux_coeff, z_coeff=z_coeff, want_logits=True,
                                      keep=True)
    bw = ops.backward_weights(w1b, w2b)
    for ga in ([1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0]):
        res = ops.moe_backward(torch.zeros_like(out), torch.tensor(ga, device=dev), x, wr_t, bw,
                               state, top_k=case.k, score_fn=score_fn, aux_coeff=aux_coeff,
                               z_coeff=z_coeff)
        xr = cpu["x"].float().clone().requires_grad_()
        wr = cpu["router"].clone().requires_grad_()
        L = xr @ wr.t()
        if score_fn == 0:
            p = L.softmax(-1)
        else:
            s = torch.sigmoid(L)
            p = s / s.sum(-1, keepdim=True)
        counts = state["counts"].cpu().float()
        lb = aux_coeff * case.E / (case.k * case.T ** 2) * (p.sum(0) * counts).sum()
        z = z_coeff * torch.logsumexp(L, -1).square().mean()
        ((ga[0] + ga[1]) * lb + (ga[0] + ga[2]) * z).backward()
        assert rel_l2(res["router"].cpu(), wr.grad) <= 1e-4, ga
        # the same router gradient in float64: the two-term bf16 split of grad_logits keeps it
        # at fp32 accuracy (each element within about 2^-17 of |g|), far inside 2e-5
        x64 = cpu["x"].double()
        w64 = cpu["router"].double().clone().requires_grad_()
        L = x64 @ w64.t()
        if score_fn == 0:
            p = L.softmax(-1)
        else:
            s = torch.sigmoid(L)
            p = s / s.sum(-1, keepdim=True)
        lb = aux_coeff * case.E / (case.k * case.T ** 2) * (p.sum(0) * counts.double()).sum()
        z = z_coeff * torch.logsumexp(L, -1).square().mean()
        ((ga[0] + ga[1]) * lb + (ga[0] + ga[2]) * z).backward()
        assert rel_l2(res["router"].cpu().double(), w64.grad) <= 2e-5, ga
        assert rel_l2(res["x"].float().cpu(), xr.grad) <= 1e-2, ga  # dx is stored in bf16
        assert float(res["w1"].float().abs().max()) == 0.0


def _recipe(**kw):
    from nexttransformer_amd.moe_recipe import MoERecipe
    base = dict(layers=4, width=256, heads=4, routed_experts=8, top_k=2, expert_width=64,
                global_batch_tokens=2048, aux_loss_coeff=0.01, z_loss_coeff=0.001)
    base.update(kw)
    return MoERecipe(**base)


def test_megatron_ffn_aux_gradient_accumulation_scale():
    """tests/test_megatron_moe.py:183-197: one backward of the full loss at aux scale 1 equals
    two backwards of half the loss at scale 0.5, and the router gradient is nonzero although
    fc2 starts at zero (so it comes from the injected aux-loss gradient alone)."""
    from nexttransformer_amd.moe import MoEFFN, set_aux_loss_scale
    r = _recipe()
    full = MoEFFN(r, 2)
    split = MoEFFN(r, 2)
    split.load_state_dict(full.state_dict())
    x = torch.randn(5, 2, 256, generator=torch.Generator().manual_seed(3)).cuda()
    try:
        set_aux_loss_scale(1.0, device="cuda")
        full(x).sum().backward()
        set_aux_loss_scale(0.5, device="cuda")
        for _ in range(2):
            (split(x).sum() / 2).backward()
        torch.testing.assert_close(full.engine.router.weight.grad,
                                   split.engine.router.weight.grad)
        assert full.engine.router.weight.grad.norm().item() > 0
    finally:
        set_aux_loss_scale(1.0)


def test_injected_aux_gradient_needs_no_aux_in_the_loss_and_skips_eval():
    """"inject": the router gradient of loss = out.sum() holds the aux term (it differs from the
    same layer with zero coefficients); in eval mode nothing is injected (MCore's router applies
    the aux loss only while training)."""
    from nexttransformer_amd.moe import MoEFFN, set_aux_loss_scale
    set_aux_loss_scale(1.0)
    x = torch.randn(3, 40, 256, generator=torch.Generator().manual_seed(4)).cuda()

    def router_grad(recipe, train=True):
        m = MoEFFN(recipe, 2)
        _randomise_fc2(m.engine, 5)
        m.train(train)
        (m(x).float().square().sum() * 1e-3).backward()  # small beside the aux term
        return m.engine.router.weight.grad.clone()
    with_aux = router_grad(_recipe(aux_loss_coeff=0.5, z_loss_coeff=0.1))
    without = router_grad(_recipe(aux_loss_coeff=0.0, z_loss_coeff=0.0))
    evaluated = router_grad(_recipe(aux_loss_coeff=0.5, z_loss_coeff=0.1), train=False)
    assert rel_l2(with_aux, without) > 1e-1
    torch.testing.assert_close(evaluated, without, rtol=1e-6, atol=1e-9)


def test_plugin_loss_route_and_injection_give_the_same_gradients():
    """The plugin block (aux in the loss through the shell's sum of `last_aux`, lm.py:386-388)
    and the scaling adapter's engine (aux gradient injected at scale 1) train the same layer to
    the same gradients: the aux loss is counted exactly once on both routes."""
    from nexttransformer_amd.moe import MoEFFN, set_aux_loss_scale
    from nexttransformer_amd.plugins import nt_moe
    import json
    from pathlib import Path
    spec = json.loads((Path(nt_moe.__file__).parent / "method.json").read_text())
    opts = dict(spec["options"], routed_experts=16, top_k=4, aux_loss_coeff=0.3, z_loss_coeff=0.05)
    config = SimpleNamespace(method="nt_moe", width=256, heads=4, layers=4, sequence_len=32,
                             vocab_size=128, mlp_width=1024, option=lambda n: opts[n])
    block = nt_moe.ffn(config, 1)
    adapter = MoEFFN(nt_moe.recipe(config), 2)
    _randomise_fc2(block.engine, 6)
    adapter.load_state_dict({"engine." + k: v for k, v in block.engine.state_dict().items()})
    x = torch.randn(2, 32, 256, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).cuda()
    G = torch.randn(2, 32, 256, generator=torch.Generator().manual_seed(8)).cuda()
    set_aux_loss_scale(1.0)
    y = block(x)
    aux = sum((m.last_aux for m in block.modules()
               if torch.is_tensor(getattr(m, "last_aux", None))), torch.zeros((), device="cuda"))
    assert aux.item() == block.engine.last_aux_loss.item() > 0
    ((y.float() * G).sum() + aux).backward()
    ya = adapter(x)
    assert torch.equal(ya, y)
    (ya.float() * G).sum().backward()
    for (name, p), q in zip(block.engine.named_parameters(), adapter.engine.parameters()):
        assert torch.equal(p.grad, q.grad), name


def test_adapter_from_reference_recipe_matches_oracle():
    """build_model with an object carrying exactly the reference MoERecipe's fields
    (moe_recipe.py:27-47): blocks 1.. hold MoE FFNs numbered index + 1, model.moe_recipe is that
    object, and an installed FFN's forward matches the oracle (ReLU^2 experts + one shared
    expert of width d/4, softmax top-k: the reference's layer)."""
    from torch import nn
    from nexttransformer_amd.moe import MoEFFN, build_model
    ref = SimpleNamespace(layers=3, width=256, heads=4, vocab_size=64, sequence_len=8,
                          routed_experts=16, top_k=4, expert_width=64, seed=42,
                          global_batch_tokens=32, training_flops=10**20, cell_id="",
                          aux_loss_coeff=0.01, z_loss_coeff=0.001, router_init_std=0.02,
                          family="moe", unique_layers=3, loops=1)

    def backbone(recipe, device):
        model = nn.Module()
        model.transformer = nn.Module()
        model.transformer.h = nn.ModuleList()
        for _ in range(recipe.layers):
            block = nn.Module()
            block.mlp = nn.Linear(recipe.width, recipe.width, device=device)
            model.transformer.h.append(block)
        return model
    model = build_model(ref, pg_collection=None, backbone=backbone)
    assert model.moe_recipe is ref and model.moe_cpu_math is False
    assert isinstance(model.transformer.h[0].mlp, nn.Linear)
    ffn = model.transformer.h[2].mlp
    assert isinstance(ffn, MoEFFN) and ffn.engine.layer_number == 3
    _randomise_fc2(ffn.engine, 9)
    hidden = torch.randn(2, 50, 256, generator=torch.Generator().manual_seed(10))
    hidden = hidden.to(torch.bfloat16).cuda()
    with torch.no_grad():
        out = ffn(hidden)
    want = _oracle_for(ffn.engine, hidden)
    assert rel_l2(out.float().reshape(-1, 256), want["out"]) <= 1e-2
    assert torch.equal(ffn.engine.last_load.cpu(), want["counts"].long())


# the reference's debug recipe (moe_recipe.py:128-133: width 32, 2 heads, 8 experts, top-2,
# expert width 8; ReLU^2 with one shared expert of width 8) trains zero-padded to 64
DEBUG_RECIPE = dict(layers=3, width=32, heads=2, vocab_size=64, sequence_len=8, routed_experts=8,
                    top_k=2, expert_width=8, global_batch_tokens=32)


@pytest.mark.parametrize("kw", [
    dict(),
    dict(activation="swiglu", score_function="sigmoid", shared_experts=0, expert_width=128,
         allow_any_expert_width=True),
    DEBUG_RECIPE,
    dict(DEBUG_RECIPE, activation="swiglu", expert_width=24, allow_any_expert_width=True,
         shared_expert_width=40),
], ids=["relu2-shared", "swiglu-sigmoid", "debug-recipe", "debug-swiglu-odd-widths"])
def test_module_training_gradients_match_fp32_autograd(kw):
    """Every parameter's .grad and hidden.grad from MoELayer (loss mode) against fp32 autograd
    of the layer restated in PyTorch with the same selection: checks the training glue (expert
    stacking order, router transpose, dtype casts, aux feeding grad_aux)."""
    from nexttransformer_amd.moe import MoELayer
    r = _recipe(**kw)
    m = MoELayer(r, 2, aux_grad="loss")
    _randomise_fc2(m, 11)
    g = torch.Generator().manual_seed(12)
    hidden = torch.randn(2, 150, r.width, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    G = torch.randn(300, r.width, generator=g).to(torch.bfloat16)
    out, aux = m(hidden)
    g_aux = 3.0
    ((out.float().reshape(-1, r.width) * G.cuda().float()).sum() + g_aux * aux).backward()
    experts = list(m.experts.local_experts)
    stack = lambda name: torch.stack([getattr(e, name).weight.detach().cpu() for e in experts])
    sw1 = sw2 = None
    if m.shared_experts is not None:
        sw1 = m.shared_experts.linear_fc1.weight.detach().cpu()[None]
        sw2 = m.shared_experts.linear_fc2.weight.detach().cpu()[None]
    case = Case("module", 300, r.width, r.routed_experts, r.top_k, r.expert_width,
                score_fn=0 if r.score_function == "softmax" else 1,
                activation=0 if r.activation == "swiglu" else 1,
                shared_H=r.shared_expert_width if sw1 is not None else 0)
    ids = orc.topk(orc.router_logits_fixed(hidden.detach().reshape(-1, r.width).cpu(),
                                           m.router.weight.detach().cpu()), r.top_k,
                   case.score_fn)[0]
    ref = reference_grads(hidden.detach().reshape(-1, r.width).cpu(),
                          m.router.weight.detach().cpu(), None, stack("linear_fc1"),
                          stack("linear_fc2"), sw1, sw2, ids, G.float(), g_aux, case,
                          r.aux_loss_coeff, r.z_loss_coeff)
    x_ref, router_ref, w1_ref, w2_ref = ref[:4]
    assert rel_l2(hidden.grad.float().reshape(-1, r.width).cpu(), x_ref) <= 2e-2
    assert rel_l2(m.router.weight.grad.cpu(), router_ref) <= 2e-2
    for i, e in enumerate(experts):
        if w1_ref[i].norm() > 0:
            assert rel_l2(e.linear_fc1.weight.grad.cpu(), w1_ref[i]) <= 2e-2, i
        else:
            assert float(e.linear_fc1.weight.grad.abs().max()) == 0.0, i
        assert rel_l2(e.linear_fc2.weight.grad.cpu(), w2_ref[i]) <= 2e-2, i
    if sw1 is not None:
        assert rel_l2(m.shared_experts.linear_fc1.weight.grad.cpu(), ref[4][0]) <= 2e-2
        assert rel_l2(m.shared_experts.linear_fc2.weight.grad.cpu(), ref[5][0]) <= 2e-2
    assert all(p.grad.dtype == torch.float32 for p in m.parameters())


def test_module_empty_batch_trains():
    """A batch of no tokens in training mode: the forward returns an empty output and the
    backward zero gradients of the masters' shapes (fp32), for both expert-gradient modes."""
    from nexttransformer_amd.moe import MoELayer
    for mode in ("accumulate", "autograd"):
        m = MoELayer(_recipe(), 2, expert_grad=mode)
        m.train()
        hidden = torch.zeros(0, m.recipe.width, device="cuda", dtype=torch.bfloat16,
                             requires_grad=True)
        out, aux = m(hidden)
        assert out.shape == (0, m.recipe.width)
        (out.float().sum() + aux).backward()
        assert hidden.grad is not None and hidden.grad.shape == hidden.shape
        for name, p in m.named_parameters():
            assert p.grad is not None and p.grad.shape == p.shape, (mode, name)
            assert p.grad.dtype == torch.float32 and float(p.grad.abs().max()) == 0.0, (mode, name)


def test_expert_grad_modes():
    """expert_grad="autograd" hands the routed experts' gradients to autograd: the same values as
    the default mode's .grad, torch.autograd.grad can name the expert weights, and
    backward(inputs=[hidden]) leaves them alone (which the default mode does not)."""
    from nexttransformer_amd.moe import MoELayer
    r = _recipe(activation="swiglu", shared_experts=1, expert_width=128,
                allow_any_expert_width=True)
    a = MoELayer(r, 2, aux_grad="loss")
    _randomise_fc2(a, 5)
    b = MoELayer(r, 2, aux_grad="loss", expert_grad="autograd")
    b.load_state_dict(a.state_dict())
    g = torch.Generator().manual_seed(6)
    hidden = torch.randn(300, r.width, generator=g).to(torch.bfloat16).cuda()
    G = torch.randn(300, r.width, generator=g).to(torch.bfloat16).cuda()
    loss = lambda m, h: (m(h)[0].float() * G.float()).sum() + m.last_aux_loss
    loss(a, hidden).backward()
    fc1 = [e.linear_fc1.weight for e in b.experts.local_experts]
    grads = torch.autograd.grad(loss(b, hidden), fc1)
    for ea, gb in zip(a.experts.local_experts, grads):
        assert torch.equal(ea.linear_fc1.weight.grad, gb)
    # backward restricted to hidden: autograd mode leaves the experts' .grad unset
    h = hidden.clone().requires_grad_()
    loss(b, h).backward(inputs=[h])
    assert h.grad is not None
    assert all(w.grad is None for w in fc1)


def test_invalidate_weights_after_data_write():
    """The operand cache follows version counters: an optimizer step is picked up by itself; a
    write through .data (which bypasses the counter) after invalidate_weights()."""
    from nexttransformer_amd.moe import MoELayer
    r = _recipe()
    m = MoELayer(r, 2, aux_grad="loss")
    _randomise_fc2(m, 9)
    ref = MoELayer(r, 2, aux_grad="loss")
    g = torch.Generator().manual_seed(10)
    hidden = torch.randn(200, r.width, generator=g).to(torch.bfloat16).cuda().requires_grad_()

    def same_as_fresh_copy():
        ref.load_state_dict(m.state_dict())
        ref.invalidate_weights()
        return torch.equal(m(hidden)[0].view(torch.int16), ref(hidden)[0].view(torch.int16))

    m(hidden)[0].float().sum().backward()  # builds the cache
    opt = torch.optim.SGD(m.parameters(), lr=0.5)
    opt.step()
    assert same_as_fresh_copy()
    w = m.experts.local_experts[0].linear_fc2.weight
    w.data.add_(0.25)
    m.invalidate_weights()
    assert same_as_fresh_copy()
