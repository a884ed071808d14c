"""nt_moe: the MoE layer as an `ffn` plugin (nexttransformer/models/plugins.py:14, lm.py:65).

ffn(config, layer) returns a module called as module(x) with x = norm(h) [B, S, d] that returns
[B, S, d] (backbone.py:150-153) and keeps its aux loss in the tensor attribute `last_aux`, which
the shell sums into the training loss (lm.py:386-388). The shell's check requires every block's
mlp.c_fc and mlp.c_proj to be nn.Linear and initialises them (plugins.py:138-146,
backbone.py:231-232): here they are the shared expert's fc1 and fc2, the same modules as
engine.shared_experts.linear_fc1/2. Every block is an MoE block; the layer's seeds follow the
scaling adapter's numbering (layer_number = layer + 1, megatron_moe.py:199-201).
Options: routed_experts, top_k, expert_width (0 = width // 4), score_function, activation,
aux_loss_coeff, z_loss_coeff, router_init_std, seed.
"""
from torch import nn

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


class MoEBlockFFN(nn.Module):
    def __init__(self, config, layer, *, device=None):
        super().__init__()
        self.engine = MoELayer(recipe(config), layer + 1, device=device)
        self.c_fc = self.engine.shared_experts.linear_fc1
        self.c_proj = self.engine.shared_experts.linear_fc2
        self.last_aux = None

    def forward(self, x):
        out, aux = self.engine(x)
        self.last_aux = aux
        return out


def ffn(config, layer):
    return MoEBlockFFN(config, layer)


def check(config):
    recipe(config)
