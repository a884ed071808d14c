"""Host-side checks that need no GPU: the C ABI library's exports and argument validation, the
recipe mirror, the MoE module's parameter contract and initialisation, and the plugin package.

Reference anchors: nexttransformer/scaling/moe_recipe.py:26-154 and tests/test_megatron_moe.py
(recipe validation, counts), megatron_moe.py:27-29,105-120,124-182 (module contract and init),
nexttransformer/models/plugins.py:56-78,138-146 (plugin declaration rules, shell linears).
"""
import ctypes
from dataclasses import replace
import json
import re
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
from torch import nn

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nt_moe.h"


# ---------------------------------------------------------------------------------------------
# C ABI

@pytest.fixture(scope="module")
def lib():
    from nexttransformer_amd import _native
    if not _native.LIB_PATH.exists():
        pytest.skip("libnt_moe.so is not built (run __graft_entry__.build())")
    return _native.load()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(nt_moe_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_functions():
    from nexttransformer_amd import _native
    assert declared_functions() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert getattr(lib, name) is not None, name
    assert lib.nt_moe_abi_version() == 1


def test_header_constants_match_binding():
    from nexttransformer_amd import _native as nat
    text = HEADER.read_text()
    const = dict((m.group(1), int(m.group(2))) for m in
                 re.finditer(r"#define\s+NT_MOE_(\w+)\s+\(?(-?\d+)\)?", text))
    assert const["ABI_VERSION"] == nat.ABI_VERSION
    assert const["MAX_EXPERTS"] == nat.MAX_EXPERTS and const["MAX_TOPK"] == nat.MAX_TOPK
    assert const["MAX_SEGMENTS"] == nat.MAX_SEGMENTS and const["ROUTE_BLOCK"] == nat.ROUTE_BLOCK
    assert const["EINVAL"] == nat.NT_MOE_EINVAL and const["ENOSPC"] == nat.NT_MOE_ENOSPC


def test_workspace_queries(lib):
    assert lib.nt_moe_grouped_gemm_workspace_bytes() == 256
    # ranks (T*k int32, 256-aligned) + per-block counts
    assert lib.nt_moe_route_workspace_bytes(16384, 4, 32) >= 16384 * 4 * 4
    assert lib.nt_moe_route_workspace_bytes(-1, 4, 32) == 0


@pytest.mark.parametrize("T,d,E,k,score,msg", [
    (10, 64, 0, 1, 0, "E must be"),
    (10, 64, 300, 2, 0, "E must be"),
    (10, 64, 4, 5, 0, "top-k"),
    (10, 64, 16, 9, 0, "top-k"),
    (-1, 64, 4, 2, 0, "T must be"),
    (10, 12, 4, 2, 0, "multiple of 8"),
    (10, 64, 4, 2, 7, "score_fn"),
])
def test_router_argument_errors_are_einval(lib, T, d, E, k, score, msg):
    from nexttransformer_amd import _native as nat
    st = lib.nt_moe_router_fwd(None, d, None, None, T, d, E, k, score, None, None, None, None,
                               None, None, 0, None)
    assert st == nat.NT_MOE_EINVAL
    assert msg in lib.nt_moe_last_error().decode()
    with pytest.raises(ValueError, match=msg):
        nat.check(st, "router")


def test_gemm_argument_errors_are_einval(lib):
    from nexttransformer_amd import _native as nat
    st = lib.nt_moe_grouped_gemm_bf16(None, 100, 8, None, None, 1, 8, None, 100, 64, 2, None,
                                      None, 0, None)
    assert st == nat.NT_MOE_EINVAL and "K must be" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_grouped_gemm_bf16(None, 128, 8, None, None, 0, 8, None, 128, 64, 2, None,
                                      None, 0, None)
    assert st == nat.NT_MOE_EINVAL
    st = lib.nt_moe_grouped_ffn_bf16(None, 128, 8, None, None, 1, 8, None, None, 128, 100, 0,
                                     None, None, None, 0, None)
    assert st == nat.NT_MOE_EINVAL and "H must be" in lib.nt_moe_last_error().decode()


def test_backward_argument_errors_are_einval(lib):
    """The backward entry points validate shapes before touching any buffer."""
    from nexttransformer_amd import _native as nat
    st = lib.nt_moe_combine_bwd(None, 100, None, None, None, None, 4, 100, 2, None, None, None)
    assert st == nat.NT_MOE_EINVAL and "d must be" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_combine_bwd(None, 64, None, None, None, None, 4, 64, 9, None, None, None)
    assert st == nat.NT_MOE_EINVAL and "top-k" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_act_bwd(None, None, 4, 12, nat.ACT_SWIGLU, None, None)
    assert st == nat.NT_MOE_EINVAL and "H must be" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_act_bwd(None, None, 4, 16, 7, None, None)
    assert st == nat.NT_MOE_EINVAL and "activation" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_router_bwd(None, None, None, None, None, 4, 300, 2, 0, None, 0.01, 0.001,
                               None, None)
    assert st == nat.NT_MOE_EINVAL and "E must be" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_grouped_wgrad_bf16(None, 256, None, 256, 8, None, None, 1, 8, 256, 96, None,
                                       None)
    assert st == nat.NT_MOE_EINVAL and "multiples of 64" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_grouped_gemm_bf16_packed_keep(None, 256, 8, None, None, 1, 8, None, 256, 64,
                                                  nat.EPI_NONE, None, None, None)
    assert st == nat.NT_MOE_EINVAL and "SWIGLU or RELU2" in lib.nt_moe_last_error().decode()
    # the paired weight gradient checks each product's widths and buffers
    st = lib.nt_moe_grouped_wgrad_pair(None, 256, None, 256, 8, None, 256, 96, None, None, 256,
                                       None, 256, 8, None, 256, 256, None, None, 1, 8, 1, None)
    assert st == nat.NT_MOE_EINVAL and "multiples of 64" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_grouped_wgrad_pair(None, 256, None, 256, 8, None, 256, 256, None, None, 256,
                                       None, 256, 8, None, 256, 256, None, None, 1, 8, 1, None)
    assert st == nat.NT_MOE_EINVAL and "null buffer" in lib.nt_moe_last_error().decode()
    # router operands: shapes, then the first operand's layout
    st = lib.nt_moe_router_operands(None, 64, 8, 64, 32, None, 0, 0, None, None, 32, 128, None)
    assert st == nat.NT_MOE_EINVAL and "d <= dp" in lib.nt_moe_last_error().decode()
    st = lib.nt_moe_router_operands(None, 64, 8, 64, 64, None, 0, 0, None, None, 32, 128, None)
    assert st == nat.NT_MOE_EINVAL and "null" in lib.nt_moe_last_error().decode()


def test_ops_reject_cpu_tensors():
    from nexttransformer_amd import ops
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        ops.router(x, torch.zeros(64, 4), None, 2, 0, False)
    with pytest.raises(ValueError, match="GPU only"):
        ops.route_plan(torch.zeros(4, 2, dtype=torch.int32), torch.zeros(4, 2), 4, None, False)
    with pytest.raises(ValueError, match="GPU only"):
        ops.act_bwd(torch.zeros(4, 32, dtype=torch.bfloat16), torch.zeros(4, 16, dtype=torch.bfloat16), 0)
    with pytest.raises(ValueError, match="GPU only"):
        ops.grouped_wgrad(x, x, None, torch.zeros(2, dtype=torch.int32), 4)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from nexttransformer_amd import _native
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "missing.so")
    monkeypatch.setattr(_native, "_LIB", None)
    with pytest.raises(_native.NativeLibraryMissing):
        _native.load()


# ---------------------------------------------------------------------------------------------
# recipe

def t3_recipe(cell="moe-T3-L20"):
    from nexttransformer_amd.moe_recipe import load_t3_recipe
    return load_t3_recipe(cell, ROOT / "tests" / "golden" / "t3_expert_cells.json")


def test_recipe_counts_match_reference_test():
    """tests/test_megatron_moe.py:51-59: the registered cell's parameter counts and the shapes
    the recipe rejects."""
    from nexttransformer_amd.moe_recipe import MoERecipe
    r = t3_recipe()
    assert r.counts()["block_total"] == 4150558720
    assert r.counts()["block_active"] == 290488320
    assert r.counts()["model_total"] == (r.counts()["block_total"]
                                         + r.counts()["embedding_and_head"] + 2 * r.layers + 26)
    with pytest.raises(ValueError):
        replace(r, top_k=257)
    with pytest.raises(ValueError):
        replace(r, expert_width=640)
    with pytest.raises(ValueError):
        replace(r, family="dense")
    with pytest.raises(ValueError):
        t3_recipe("dense-T3-L20")
    assert isinstance(r, MoERecipe) and r.activation == "relu2" and r.shared_experts == 1
    assert (r.width, r.routed_experts, r.top_k, r.expert_width, r.layers) == (1280, 256, 8, 320, 20)


def test_recipe_counts_by_enumerating_the_stack():
    """counts() against a sum over the tensors of the stack it describes, for a SwiGLU recipe
    with a wider shared expert (so the activation and shared width terms are exercised)."""
    from nexttransformer_amd.moe_recipe import MoERecipe
    r = MoERecipe(layers=5, width=96, heads=4, vocab_size=1000, routed_experts=6, top_k=2,
                  expert_width=40, activation="swiglu", shared_expert_width=56,
                  allow_any_expert_width=True, global_batch_tokens=4096)
    d = 96
    attn = [(d, d)] * 4
    dense = [(4 * d, d), (d, 4 * d)]
    expert = lambda h: [(2 * h, d), (d, h)]
    moe = sum((expert(40) for _ in range(6)), []) + expert(56) + [(6, d)]
    used = sum((expert(40) for _ in range(2)), []) + expert(56) + [(6, d)]
    n = lambda shapes: sum(a * b for a, b in shapes)
    total = 5 * n(attn) + n(dense) + 4 * n(moe)
    active = 5 * n(attn) + n(dense) + 4 * n(used)
    c = r.counts()
    assert (c["block_total"], c["block_active"]) == (total, active)
    assert c["embedding_and_head"] == 2 * d * 1024
    assert r.moe_layer_params() == n(moe)


def test_t3_cells_read_their_family_recipe():
    """Every expert cell of the manifest loads with its family's expert counts and activation;
    a family that changes them is followed (read, not assumed), and one this build cannot run
    is rejected."""
    data = json.loads((ROOT / "tests" / "golden" / "t3_expert_cells.json").read_text())
    for cell in data["cells"]:
        r = t3_recipe(cell["id"])
        assert (r.routed_experts, r.top_k, r.shared_experts, r.activation) == (256, 8, 1, "relu2")
        assert (r.layers, r.width, r.expert_width, r.family) == (
            cell["layers"], cell["width"], cell["expertWidth"], cell["family"])
    looped, moe = t3_recipe("looped-T3-L20"), t3_recipe("moe-T3-L20")
    assert looped.layers == moe.layers and looped.unique_layers < looped.layers
    with pytest.raises(ValueError):
        looped.counts()
    with pytest.raises(ValueError):
        t3_recipe("kda-dsa-T3-L20").counts()
    import tempfile
    from nexttransformer_amd.moe_recipe import load_t3_recipe
    with tempfile.TemporaryDirectory() as tmp:
        def variant(**change):
            copy = json.loads(json.dumps(data))
            next(f for f in copy["families"] if f["id"] == "moe")["recipe"].update(change)
            path = Path(tmp) / "t3.json"
            path.write_text(json.dumps(copy))
            return path
        assert load_t3_recipe("moe-T3-L20", variant(selectedExperts=4)).top_k == 4
        with pytest.raises(ValueError, match="expert FFN"):
            load_t3_recipe("moe-T3-L20", variant(ffn="GELU"))
        with pytest.raises(ValueError, match="dense"):
            load_t3_recipe("moe-T3-L20", variant(firstLayerDense=False))


@pytest.mark.parametrize("change,msg", [
    (dict(score_function="topk"), "score_function"),
    (dict(activation="gelu"), "activation"),
    (dict(expert_dtype="fp16"), "expert_dtype"),
    (dict(shared_experts=2), "shared_experts"),
    (dict(aux_loss_coeff=-1.0), "aux_loss_coeff"),
    (dict(z_loss_coeff=float("nan")), "z_loss_coeff"),
    (dict(router_init_std=0.0), "router_init_std"),
    (dict(global_batch_tokens=100), "whole number of sequences"),
    (dict(heads=3), "divisible"),
    (dict(layers=1, unique_layers=1), "at least two layers"),
    (dict(top_k=0), "top_k"),
])
def test_recipe_rejects_invalid_values(change, msg):
    with pytest.raises(ValueError, match=msg):
        replace(t3_recipe(), **change)


def test_recipe_added_keys():
    from nexttransformer_amd.moe_recipe import MoERecipe
    r = MoERecipe(layers=4, width=1024, heads=8, routed_experts=32, top_k=4, expert_width=512,
                  activation="swiglu", shared_experts=0, allow_any_expert_width=True,
                  global_batch_tokens=16384)
    assert r.fc1_rows == 1024 and r.expert_params() == 1024 * 1024 + 1024 * 512
    assert r.moe_layer_params() == 32 * r.expert_params() + 1024 * 32
    assert MoERecipe(layers=3, width=32, heads=2).shared_expert_width == 8


def _reference_shaped_recipe(**values):
    """An object carrying exactly the reference MoERecipe's fields
    (nexttransformer/scaling/moe_recipe.py:27-47) and nothing of this build's."""
    from types import SimpleNamespace
    base = dict(layers=3, width=32, heads=2, vocab_size=64, sequence_len=8, routed_experts=8,
                top_k=2, expert_width=8, seed=42, global_batch_tokens=32,
                training_flops=10**20, cell_id="moe-T3-L20-cpu-debug", aux_loss_coeff=0.01,
                z_loss_coeff=0.001, router_init_std=0.02, family="moe", unique_layers=3,
                loops=1)
    base.update(values)
    return SimpleNamespace(**base)


def test_recipe_from_reference_fields():
    """A reference recipe converts field by field; the build keys take the reference layer's
    values (ReLU^2, softmax, bf16, one shared expert of the routed width)."""
    from nexttransformer_amd.moe_recipe import MoERecipe
    ref = _reference_shaped_recipe()
    r = MoERecipe.from_any(ref)
    for name in vars(ref):
        assert getattr(r, name) == getattr(ref, name), name
    assert (r.activation, r.score_function, r.expert_dtype, r.shared_experts,
            r.shared_expert_width) == ("relu2", "softmax", "bf16", 1, 8)
    assert MoERecipe.from_any(r) is r
    with pytest.raises(ValueError, match="lacks"):
        MoERecipe.from_any(object())
    with pytest.raises(ValueError):
        MoERecipe.from_any(_reference_shaped_recipe(top_k=9))


# ---------------------------------------------------------------------------------------------
# MoE module (constructed on the CPU; its forward needs the GPU)

def small_recipe(**kw):
    from nexttransformer_amd.moe_recipe import MoERecipe
    base = dict(layers=4, width=64, heads=4, routed_experts=8, top_k=2, expert_width=16,
                global_batch_tokens=2048)
    base.update(kw)
    return MoERecipe(**base)


def test_module_parameter_names_and_shapes():
    """Names of tests/test_megatron_moe.py:104-112,138-141; fp32 masters."""
    from nexttransformer_amd.moe import MoELayer
    r = small_recipe()
    m = MoELayer(r, 2, device="cpu")
    shapes = {n: tuple(p.shape) for n, p in m.named_parameters()}
    assert shapes["router.weight"] == (8, 64)
    for i in range(8):
        assert shapes[f"experts.local_experts.{i}.linear_fc1.weight"] == (16, 64)
        assert shapes[f"experts.local_experts.{i}.linear_fc2.weight"] == (64, 16)
    assert shapes["shared_experts.linear_fc1.weight"] == (16, 64)
    assert shapes["shared_experts.linear_fc2.weight"] == (64, 16)
    assert len(shapes) == 1 + 2 * 8 + 2
    assert all(p.dtype == torch.float32 for p in m.parameters())
    assert sum(p.numel() for p in m.parameters()) == r.moe_layer_params()
    g = MoELayer(small_recipe(activation="swiglu", shared_experts=0), 2, device="cpu")
    assert g.experts.local_experts[0].linear_fc1.weight.shape == (32, 64)
    assert g.shared_experts is None


def test_module_init_follows_reference_seeding():
    """megatron_moe.py:105-120 on the CPU: fork_rng + manual_seed(seed + 100003 layer + id),
    fc1 ~ U(+-0.4 sqrt(3/d)) (:27-29), fc2 zero, router N(0, std) with id E + 1."""
    from nexttransformer_amd.moe import MoELayer
    r = small_recipe(seed=7)
    layer = 3
    m = MoELayer(r, layer, device="cpu")
    base = r.seed + 100003 * layer

    def reference_fc1(shape, seed):
        with torch.random.fork_rng(devices=[]):
            torch.manual_seed(seed)
            w = torch.empty(shape)
            bound = 0.4 * (3 / shape[-1]) ** 0.5
            return nn.init.uniform_(w, -bound, bound)

    for i, e in enumerate(m.experts.local_experts):
        assert torch.equal(e.linear_fc1.weight, reference_fc1((16, 64), base + i)), i
        assert not e.linear_fc2.weight.any()
    assert torch.equal(m.shared_experts.linear_fc1.weight, reference_fc1((16, 64), base + 8))
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(base + 8 + 1)
        router = nn.init.normal_(torch.empty(8, 64), std=r.router_init_std)
    assert torch.equal(m.router.weight, router)
    # the module leaves the caller's RNG stream alone
    torch.manual_seed(123)
    a = torch.rand(3)
    torch.manual_seed(123)
    MoELayer(r, layer, device="cpu")
    assert torch.equal(torch.rand(3), a)


def test_module_state_dict_round_trip_and_repack():
    from nexttransformer_amd.moe import MoELayer
    a = MoELayer(small_recipe(), 2, device="cpu")
    b = MoELayer(small_recipe(seed=99), 2, device="cpu")
    b.load_state_dict(a.state_dict())
    for (n, p), (_, q) in zip(a.named_parameters(), b.named_parameters()):
        assert torch.equal(p, q), n
    packed = b.packed_weights()
    assert b.packed_weights() is packed  # unchanged masters: cached
    with torch.no_grad():
        b.experts.local_experts[3].linear_fc2.weight.add_(1.0)
    repacked = b.packed_weights()
    assert repacked is not packed
    fc2 = b.experts.local_experts[3].linear_fc2.weight.to(torch.bfloat16)
    assert torch.equal(repacked["w2"][3][:, :16], fc2)  # hidden 16 is zero-padded to 64
    assert not repacked["w2"][3][:, 16:].any()


@pytest.mark.parametrize("activation", ["swiglu", "relu2"])
def test_padded_packing_computes_the_same_layer(activation):
    """Widths that are not multiples of 64 are zero-padded for the GEMM tiles; the padded
    weights must give the same expert outputs (checked in fp64 with the oracle's experts)."""
    from nexttransformer_amd.moe import MoELayer
    from oracle import moe_oracle as orc
    r = small_recipe(width=40, heads=4, expert_width=24, activation=activation,
                     allow_any_expert_width=True)
    m = MoELayer(r, 2, device="cpu")
    with torch.no_grad():
        for e in [*m.experts.local_experts, m.shared_experts]:
            e.linear_fc2.weight.normal_(0, 0.1)
    p = m.packed_weights()
    assert p["router_t"].shape == (64, 8) and p["w1"].shape[2] == 64 and p["w2"].shape[1:] == (64, 64)
    act = orc.SWIGLU if activation == "swiglu" else orc.RELU2
    x = torch.randn(10, 40, dtype=torch.float64)
    xp = torch.nn.functional.pad(x, (0, 24))
    for i, e in enumerate(m.experts.local_experts):
        ref = orc.expert_ffn(x, e.linear_fc1.weight.to(torch.bfloat16).double(),
                             e.linear_fc2.weight.to(torch.bfloat16).double(), act)
        got = orc.expert_ffn(xp, p["w1"][i].double(), p["w2"][i].double(), act)
        assert torch.allclose(got[:, :40], ref, rtol=1e-12, atol=1e-14) and not got[:, 40:].any()
    assert torch.equal(xp.float() @ p["router_t"], x.float() @ m.router.weight.t())


def test_module_errors():
    from nexttransformer_amd.moe import MoEFFN, MoELayer
    r = small_recipe()
    with pytest.raises(ValueError, match="one GPU"):
        MoELayer(r, 2, SimpleNamespace(ep=SimpleNamespace(size=lambda: 8)), device="cpu")
    with pytest.raises(ValueError, match="CPU math"):
        MoEFFN(r, 2, cpu_math=True, device="cpu")
    with pytest.raises(ValueError, match="GPU only"):  # fp8 packing quantises on the GPU
        MoELayer(small_recipe(expert_dtype="fp8"), 2, device="cpu").packed_weights()
    m = MoELayer(r, 2, device="cpu")
    with pytest.raises(ValueError, match="GPU only"):
        with torch.no_grad():
            m(torch.zeros(2, 3, 64))
    with pytest.raises(ValueError, match="width"):
        m(torch.zeros(2, 3, 32))


# ---------------------------------------------------------------------------------------------
# plugin package

PLUGIN = ROOT / "nexttransformer_amd" / "plugins" / "nt_moe"


def test_plugin_declaration_follows_registry_rules():
    """The checks of plugins.discover (plugins.py:56-78), restated."""
    spec = json.loads((PLUGIN / "method.json").read_text())
    name_re = re.compile(r"[a-z][a-z0-9_]{1,40}")
    scalar = lambda v: isinstance(v, (str, int, float, bool)) or (
        isinstance(v, list) and all(scalar(i) for i in v))
    assert name_re.fullmatch(spec["name"]) and spec["name"] == PLUGIN.name
    assert spec["family"] in ("looped", "sparse", "linear", "residual", "hybrid", "others")
    assert all(name_re.fullmatch(k) and scalar(v) for k, v in spec["options"].items())
    assert set(spec.get("debug_options", {})) <= set(spec["options"])
    assert set(spec.get("shell", {})) <= {"layers", "mlp_width", "window_pattern"}
    assert isinstance(spec.get("layer_multiple", 1), int) and spec.get("layer_multiple", 1) > 0
    assert (PLUGIN / "__init__.py").is_file()


def plugin_config(**options):
    spec = json.loads((PLUGIN / "method.json").read_text())
    opts = dict(spec["options"], **options)
    return SimpleNamespace(method="nt_moe", width=64, heads=4, layers=4, sequence_len=32,
                           vocab_size=128, mlp_width=256, option=lambda n: opts[n])


def test_plugin_ffn_exposes_shell_linears():
    import importlib
    plugin = importlib.import_module("nexttransformer_amd.plugins.nt_moe")
    config = plugin_config()
    plugin.check(config)
    module = plugin.MoEBlockFFN(config, 0, device="cpu")
    assert isinstance(module.c_fc, nn.Linear) and isinstance(module.c_proj, nn.Linear)
    assert module.c_fc is module.engine.shared_experts.linear_fc1
    assert module.c_proj is module.engine.shared_experts.linear_fc2
    assert module.engine.layer_number == 1 and module.engine.recipe.expert_width == 16
    names = [n for n, _ in module.named_parameters()]
    assert "engine.router.weight" in names and len(names) == len(set(names))
    with pytest.raises(ValueError):
        plugin.check(plugin_config(top_k=99))
    with pytest.raises(ValueError):
        plugin.check(plugin_config(activation="gelu"))


def test_plugin_first_layer_dense_and_one_last_aux_per_block():
    """The T3 families keep layer 0 dense (reference_blocks.py:48-58); with the option on, the
    plugin's layer 0 is a dense ReLU^2 FFN whose c_fc / c_proj the shell can initialise. In an
    MoE block exactly one module of the subtree may expose a tensor `last_aux` -- the block --
    since the shell sums `last_aux` over all modules (lm.py:386-388)."""
    import importlib
    plugin = importlib.import_module("nexttransformer_amd.plugins.nt_moe")
    config = plugin_config()
    dense = plugin.ffn(config, 0, device="cpu")
    assert isinstance(dense, plugin.DenseBlockFFN)
    assert dense.c_fc.weight.shape == (256, 64) and dense.c_proj.weight.shape == (64, 256)
    assert isinstance(dense.c_fc, nn.Linear) and isinstance(dense.c_proj, nn.Linear)
    x = torch.randn(2, 3, 64)
    ref = torch.relu(x @ dense.c_fc.weight.t()).square() @ dense.c_proj.weight.t()
    torch.testing.assert_close(dense(x), ref)
    assert isinstance(plugin.ffn(plugin_config(first_layer_dense=False), 0, device="cpu"),
                      plugin.MoEBlockFFN)
    with pytest.raises(ValueError, match="first_layer_dense"):
        plugin.check(plugin_config(first_layer_dense="yes"))
    block = plugin.ffn(config, 2, device="cpu")
    assert block.engine.layer_number == 3 and block.engine.aux_grad == "loss"
    # what the shell's sum would see after a forward: stand the engine's forward in by a value
    block.last_aux = torch.tensor(0.5)
    block.engine.last_aux_loss = block.last_aux
    holders = [m for m in block.modules() if torch.is_tensor(getattr(m, "last_aux", None))]
    assert holders == [block]
    total = sum((m.last_aux for m in block.modules()
                 if torch.is_tensor(getattr(m, "last_aux", None))), torch.zeros(()))
    assert total.item() == 0.5


def test_install_moe_ffns_mirrors_the_scaling_adapter():
    """megatron_moe.py:203-207: blocks 1.. get MegatronFFN(recipe, index + 1), block 0 keeps its
    FFN, model.moe_recipe is the recipe as given (here reference-shaped) and moe_cpu_math is
    False; the engines inject the aux gradient and expose no `last_aux`."""
    from nexttransformer_amd.moe import MegatronFFN, MoEFFN, install_moe_ffns
    ref = _reference_shaped_recipe()

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.mlp = nn.Linear(32, 32)

    model = nn.Module()
    model.transformer = nn.Module()
    model.transformer.h = nn.ModuleList(Block() for _ in range(3))
    dense = model.transformer.h[0].mlp
    install_moe_ffns(model, ref, device="cpu")
    assert model.transformer.h[0].mlp is dense
    for i in (1, 2):
        mlp = model.transformer.h[i].mlp
        assert isinstance(mlp, MoEFFN) and MegatronFFN is MoEFFN
        assert mlp.engine.layer_number == i + 1 and mlp.engine.aux_grad == "inject"
        assert not hasattr(mlp, "last_aux") and not hasattr(mlp.engine, "last_aux")
        assert mlp.engine.recipe.routed_experts == 8 and mlp.engine.shared_experts is not None
    assert model.moe_recipe is ref and model.moe_cpu_math is False
    with pytest.raises(ValueError, match="CPU math"):
        install_moe_ffns(model, ref, cpu_math=True, device="cpu")
    # initialisation follows the global numbering: block 2's engine is layer 3's
    from nexttransformer_amd.moe import MoELayer
    twin = MoELayer(ref, 3, device="cpu")
    assert torch.equal(twin.router.weight, model.transformer.h[2].mlp.engine.router.weight)


def test_set_aux_loss_scale_value():
    from nexttransformer_amd import moe
    try:
        moe.set_aux_loss_scale(0.25)
        g = moe._injected_aux_grad(torch.device("cpu"))
        assert g.tolist() == [0.25, 0.0, 0.0]
    finally:
        moe.set_aux_loss_scale(1.0)
    assert moe._injected_aux_grad(torch.device("cpu")).tolist() == [1.0, 0.0, 0.0]
