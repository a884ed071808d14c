"""MoE recipe: the reference's MoERecipe config keys plus the keys this MI355X build adds.

Mirrors nexttransformer/scaling/moe_recipe.py:26-154 (field names, defaults, validation,
counts/estimate/manifest, load_t3_recipe and
ValueError behaviour). Added keys, all explicit so no reference recipe changes meaning:
  score_function         "softmax" (the reference's router, megatron_moe.py:43) or "sigmoid"
                         (top-k on logits, sigmoid scores normalised over the selected)
  activation             "relu2" (the reference's two-matrix ReLU^2 expert, megatron_moe.py:23-24)
                         or "swiglu" (fc1 rows [0, H) gate, [H, 2H) value: silu(g) * u, the
                         gated_linear_unit order of the MCore config the adapter builds)
  expert_dtype           "bf16" or "fp8" (e4m3 weights with 128x128 block scales)
  shared_experts         0 or 1 ungated shared expert (the reference always has 1)
  shared_expert_width    hidden width of the shared expert (default: expert_width)
  allow_any_expert_width the reference requires expert_width == width // 4
                         (moe_recipe.py:63-64); True relaxes exactly that check
"""
from dataclasses import asdict, dataclass, replace
import json
import math
from pathlib import Path

EXPERT_FAMILIES = ("moe", "looped", "kda-dsa")
FULL_ATTENTION = ("moe", "looped")
SCORE_FUNCTIONS = ("softmax", "sigmoid")
ACTIVATIONS = ("relu2", "swiglu")
EXPERT_DTYPES = ("bf16", "fp8")
# The feed-forward keys the T3 expert families share (moe_recipe.py:14-17); a manifest whose
# expert families disagree with them is rejected by load_t3_recipe.
SHARED_FFN_RECIPE = dict(firstLayerDense=True, ffn="ReLU²", routedExperts=256,
                         selectedExperts=8, sharedExperts=1, expertWidthDivisor=4)
ATTENTION_NOTE = {"moe": "native full causal MHA; no VE",
                  "looped": "native full causal MHA, shared core executed twice; no VE",
                  "kda-dsa": "three KDA mixers then one DSA mixer; no VE"}


@dataclass(frozen=True)
class MoERecipe:
    layers: int
    width: int
    heads: int
    vocab_size: int = 32768
    sequence_len: int = 2048
    routed_experts: int = 256
    top_k: int = 8
    expert_width: int | None = None
    seed: int = 42
    global_batch_tokens: int = 1048576
    training_flops: int = 10**20
    cell_id: str = ""
    aux_loss_coeff: float = 0.01
    z_loss_coeff: float = 0.001
    router_init_std: float = 0.02
    family: str = "moe"
    unique_layers: int | None = None
    loops: int = 1
    # keys added by this build
    score_function: str = "softmax"
    activation: str = "relu2"
    expert_dtype: str = "bf16"
    shared_experts: int = 1
    shared_expert_width: int | None = None
    allow_any_expert_width: bool = False

    def __post_init__(self):
        if self.expert_width is None:
            object.__setattr__(self, "expert_width", self.width // 4)
        if self.unique_layers is None:
            object.__setattr__(self, "unique_layers", self.layers)
        if self.shared_expert_width is None:
            object.__setattr__(self, "shared_expert_width", self.expert_width)
        if self.family not in EXPERT_FAMILIES:
            raise ValueError(f"not a T3 expert family: {self.family}")
        if not 2 <= self.unique_layers <= self.layers or self.loops < 1:
            raise ValueError("unique layers must be between two and the executed depth")
        if min(self.layers, self.width, self.heads, self.vocab_size, self.sequence_len,
               self.routed_experts, self.expert_width, self.global_batch_tokens,
               self.training_flops) <= 0:
            raise ValueError("model dimensions and budgets must be positive")
        if self.layers < 2 or self.width < 24 or self.width % self.heads or self.width % 4:
            raise ValueError("MoE needs >=2 layers, width>=24 divisible by heads and four")
        if (self.width // self.heads) % 2:
            raise ValueError("even head dimension is required")
        if self.expert_width != self.width // 4 and not self.allow_any_expert_width:
            raise ValueError("expert_width must be width // 4 unless allow_any_expert_width=True")
        if not 1 <= self.top_k <= self.routed_experts:
            raise ValueError("top-k must fit the expert count")
        if self.global_batch_tokens % self.sequence_len:
            raise ValueError("batch must contain whole sequences")
        if not all(math.isfinite(x) and x >= 0 for x in (self.aux_loss_coeff, self.z_loss_coeff)):
            raise ValueError("routing loss coefficients must be finite and nonnegative")
        if not math.isfinite(self.router_init_std) or self.router_init_std <= 0:
            raise ValueError("router initialization standard deviation must be positive")
        if self.score_function not in SCORE_FUNCTIONS:
            raise ValueError(f"score_function must be one of {SCORE_FUNCTIONS}")
        if self.activation not in ACTIVATIONS:
            raise ValueError(f"activation must be one of {ACTIVATIONS}")
        if self.expert_dtype not in EXPERT_DTYPES:
            raise ValueError(f"expert_dtype must be one of {EXPERT_DTYPES}")
        if self.shared_experts not in (0, 1):
            raise ValueError("shared_experts must be 0 or 1")
        if self.shared_expert_width <= 0:
            raise ValueError("shared_expert_width must be positive")

    @property
    def fc1_rows(self):
        """Rows of an expert's fc1: 2H for SwiGLU (gate, value), H for ReLU^2."""
        return 2 * self.expert_width if self.activation == "swiglu" else self.expert_width

    def expert_params(self, width=None):
        """Parameters of one expert of hidden `width` (fc1 + fc2)."""
        h = self.expert_width if width is None else width
        rows = 2 * h if self.activation == "swiglu" else h
        return rows * self.width + self.width * h

    def block_active(self):
        """Parameters a token activates across the executed depth (reference convention,
        moe_recipe.py:74-85, generalised to the expert activation and shared width)."""
        if self.family not in FULL_ATTENTION:
            raise ValueError(f"{self.family} attention needs its own cost proof")
        d, e = self.width, self.routed_experts
        shared = self.shared_experts * self.expert_params(self.shared_expert_width)
        return (4 * self.layers * d * d + 8 * d * d
                + (self.layers - 1) * (self.top_k * self.expert_params() + shared)
                + (self.layers - 1) * d * e)

    def describes_capacity(self):
        """Whether the parameter counts describe the family: a flat stack of MHA layers."""
        return self.family in FULL_ATTENTION and self.unique_layers == self.layers

    def counts(self):
        """Parameter counts (moe_recipe.py:93-106): attention 4Ld^2, a dense first FFN 8d^2,
        (L-1) MoE layers of E routed + shared experts and a d x E router, embeddings and head
        padded to 64 rows, and the backbone's 2L + 26 scalars."""
        if not self.describes_capacity():
            raise ValueError(f"{self.family} capacity needs its own accounting")
        d, e = self.width, self.routed_experts
        shared = self.shared_experts * self.expert_params(self.shared_expert_width)
        total = (4 * self.layers * d * d + 8 * d * d
                 + (self.layers - 1) * (e * self.expert_params() + shared)
                 + (self.layers - 1) * d * e)
        small = 2 * self.layers + 26
        io = 2 * d * math.ceil(self.vocab_size / 64) * 64
        return dict(block_total=total, block_active=self.block_active(), embedding_and_head=io,
                    native_small_parameters=small, model_total=total + io + small)

    def estimate(self):
        """Main-term training cost (moe_recipe.py:108-118): 6 x active parameters + attention
        12 s d L + head 6 d V FLOP per token, and the updates / tokens the budget buys."""
        if self.family not in FULL_ATTENTION:
            return dict(flops_per_token_main_term=None, estimated_updates=None,
                        estimated_tokens=None, cost_proof_complete=False)
        d, s = self.width, self.sequence_len
        flops = 6 * self.block_active() + 12 * s * d * self.layers + 6 * d * self.vocab_size
        updates = round(self.training_flops / (flops * self.global_batch_tokens))
        return dict(flops_per_token_main_term=flops, estimated_updates=updates,
                    estimated_tokens=updates * self.global_batch_tokens, cost_proof_complete=False)

    def manifest(self):
        counts = self.counts() if self.describes_capacity() else None
        act = {"relu2": "ReLU squared", "swiglu": "SwiGLU"}[self.activation]
        return dict(protocol="nextt-scale-2k-v1", recipe=asdict(self), counts=counts,
                    estimate=self.estimate(), attention=ATTENTION_NOTE[self.family],
                    ffn=f"first dense 4d; then routed top-k plus {self.shared_experts} shared; {act}",
                    gpu_validated=False, formal_training_ready=False)

    def moe_layer_params(self):
        """Parameters of one MoE layer as built by nexttransformer_amd.moe.MoELayer."""
        shared = self.shared_experts * self.expert_params(self.shared_expert_width)
        return self.routed_experts * self.expert_params() + shared + self.width * self.routed_experts

    def debug(self, *, routed_experts=8, top_k=2):
        """The reference's CPU debug shrink (moe_recipe.py:128-133)."""
        shape = (dict(layers=2 + self.loops, unique_layers=3) if self.loops > 1
                 else dict(layers=3, unique_layers=3))
        return replace(self, **shape, width=32, heads=2, vocab_size=64, sequence_len=8,
                       routed_experts=routed_experts, top_k=top_k, expert_width=8,
                       shared_expert_width=8, global_batch_tokens=32,
                       cell_id=self.cell_id + "-cpu-debug")


def load_t3_recipe(cell_id="moe-T3-L20", path=None):
    """The recipe of a T3 expert cell from a scaling manifest (moe_recipe.py:136-154).

    `path` is the manifest JSON (the reference keeps it at configs/scaling/t3.json); this
    package ships none, so it is required.
    """
    if path is None:
        raise ValueError("load_t3_recipe needs the path of a T3 scaling manifest")
    data = json.loads(Path(path).read_text())
    cell = next((c for c in data["cells"]
                 if c["id"] == cell_id and c["family"] in EXPERT_FAMILIES), None)
    if cell is None:
        raise ValueError(f"unknown T3 expert cell: {cell_id}")
    rule = next(f["recipe"] for f in data["families"] if f["id"] == cell["family"])
    if ({k: v for k, v in rule.items() if k in SHARED_FFN_RECIPE} != SHARED_FFN_RECIPE
            or data["valueEmbeddings"] or data["protocol"] != "nextt-scale-2k-v1"):
        raise ValueError("the shared T3 expert recipe changed; review the adapter before using it")
    loops = rule.get("loops", 1)
    unique = (cell["preLayers"] + cell["coreLayers"] + cell["postLayers"] if loops > 1
              else cell["layers"])
    return MoERecipe(layers=cell["layers"], width=cell["width"], heads=cell["heads"],
                     vocab_size=data["vocabSize"], sequence_len=data["sequenceLength"],
                     seed=data["seed"], global_batch_tokens=data["globalBatchTokens"],
                     training_flops=data["trainingFlops"], expert_width=cell["expertWidth"],
                     cell_id=cell_id, family=cell["family"], unique_layers=unique, loops=loops)
