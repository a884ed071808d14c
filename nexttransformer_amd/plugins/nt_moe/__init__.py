"""nt_moe: the MoE layer as an `ffn` plugin (nexttransformer/models/plugins.py:14, lm.py:65).

ffn(config, layer) returns a module called as module(x) with x = norm(h) [B, S, d] that returns
[B, S, d] (backbone.py:150-153). An MoE block keeps its aux loss in the tensor attribute
`last_aux`, which the shell sums into the training loss (lm.py:386-388); its engine therefore
runs in the "loss" aux-gradient mode (no injected gradient) and keeps its own copy under
another name, so the shell's sum over modules counts the aux loss exactly once.
The shell's check requires every block's mlp.c_fc and mlp.c_proj to be nn.Linear and
initialises them (plugins.py:138-146, backbone.py:231-232): in an MoE block they are the shared
expert's fc1 and fc2, the same modules as engine.shared_experts.linear_fc1/2.
With first_layer_dense (the T3 expert families' rule, configs/scaling/t3.json "firstLayerDense";
reference_blocks.py:48-58) layer 0 is a dense ReLU^2 FFN of width config.mlp_width instead; the
MoE layers' seeds follow the scaling adapter's numbering (layer_number = layer + 1,
megatron_moe.py:203-205).
Options: routed_experts, top_k, expert_width (0 = width // 4), score_function, activation,
aux_loss_coeff, z_loss_coeff, router_init_std, seed, first_layer_dense.
"""
import torch
from torch import nn
from torch.nn import functional as F

from nexttransformer_amd.moe import MoELayer
from nexttransformer_amd.moe_recipe import MoERecipe

OPTIONS = ("routed_experts", "top_k", "expert_width", "score_function", "activation",
           "aux_loss_coeff", "z_loss_coeff", "router_init_std", "seed")


def recipe(config):
    """The MoERecipe of a plugin config; raises ValueError for invalid option values."""
    opt = {name: config.option(name) for name in OPTIONS}
    width = config.width
    expert_width = opt.pop("expert_width") or width // 4
    return MoERecipe(layers=max(2, config.layers), width=width, heads=config.heads,
                     vocab_size=config.vocab_size, sequence_len=config.sequence_len,
                     global_batch_tokens=config.sequence_len, expert_width=expert_width,
                     shared_experts=1, shared_expert_width=expert_width,
                     allow_any_expert_width=True, cell_id=f"plugin-{config.method}", **opt)


class _MasterLinear(nn.Linear):
    """Bias-free linear whose fp32 master is cast to the input's dtype per call, as the
    backbone's Linear does (backbone.py:45-50)."""

    def forward(self, x):
        return F.linear(x, self.weight.to(x.dtype))


class DenseBlockFFN(nn.Module):
    """The dense first-layer FFN of the expert families: c_proj(relu(c_fc x)^2) with hidden
    width config.mlp_width (lm.py:29-35). Plain PyTorch: it is not part of the MoE path."""

    def __init__(self, config, *, device=None):
        super().__init__()
        self.c_fc = _MasterLinear(config.width, config.mlp_width, bias=False, device=device)
        self.c_proj = _MasterLinear(config.mlp_width, config.width, bias=False, device=device)

    def forward(self, x):
        return self.c_proj(F.relu(self.c_fc(x)).square())


class MoEBlockFFN(nn.Module):
    def __init__(self, config, layer, *, device=None):
        super().__init__()
        self.engine = MoELayer(recipe(config), layer + 1, device=device, aux_grad="loss")
        self.c_fc = self.engine.shared_experts.linear_fc1
        self.c_proj = self.engine.shared_experts.linear_fc2
        self.last_aux = None

    def forward(self, x):
        out, aux = self.engine(x)
        self.last_aux = aux
        return out


def ffn(config, layer, *, device=None):
    if layer == 0 and _first_layer_dense(config):
        return DenseBlockFFN(config, device=device)
    return MoEBlockFFN(config, layer, device=device)


def _first_layer_dense(config):
    value = config.option("first_layer_dense")
    if not isinstance(value, bool):
        raise ValueError("first_layer_dense must be true or false")
    return value


def check(config):
    recipe(config)
    _first_layer_dense(config)
