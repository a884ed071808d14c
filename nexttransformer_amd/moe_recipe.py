"""The MoE layer's configuration: the reference recipe's keys, plus the few this build adds.

Interface kept from nexttransformer/scaling/moe_recipe.py:26-47 (so a recipe means the same in
both code bases): the field names and their defaults, expert_width defaulting to width // 4,
unique_layers defaulting to layers, and ValueError for a configuration that cannot be built.
Everything else here is this build's own: the checks are grouped by what they protect (shape,
routing, numerics, build keys), and the reference's cost estimates, manifest and CPU-debug
shrink are not carried over (the MoE layer does not use them). counts() stays, because the
reference optimizer reads block_total and embedding_and_head from model.moe_recipe
(nexttransformer/scaling/megatron_optimizer.py:60-65).

Keys this build adds (all optional; a reference recipe keeps its meaning):
  score_function   "softmax" (top-k on the logits, softmax over the selected: the reference's
                   router, megatron_moe.py:43) or "sigmoid" (sigmoid scores of the selected,
                   normalised over them)
  activation       "relu2" (the reference's two-matrix expert, megatron_moe.py:23-24) or
                   "swiglu" (fc1 rows [0, H) are the gate, [H, 2H) the value: silu(g) * u)
  expert_dtype     "bf16" or "fp8" (e4m3 expert weights with 128 x 128 block scales)
  shared_experts   0 or 1 always-on ungated expert (the reference always has 1)
  shared_expert_width       its hidden width (default: expert_width)
  allow_any_expert_width    the reference fixes expert_width = width // 4; True lifts that
"""
from dataclasses import dataclass, fields
import json
import math
from pathlib import Path

SCORE_FUNCTIONS = ("softmax", "sigmoid")
ACTIVATIONS = ("relu2", "swiglu")
EXPERT_DTYPES = ("bf16", "fp8")
# Families of the reference's T3 scaling study that put routed experts in their FFNs, and the
# ones among them whose attention is plain full MHA (parameter counts apply only to those).
EXPERT_FAMILIES = ("moe", "looped", "kda-dsa")
MHA_FAMILIES = ("moe", "looped")
# Parameters of the native backbone outside the blocks and the vocabulary matrices: one
# residual and one x0 scalar per layer plus 26 fixed gate / mixing scalars.
_BACKBONE_SCALARS_PER_LAYER = 2
_BACKBONE_SCALARS_FIXED = 26
# Manifest spelling of the expert activation -> the recipe's.
_MANIFEST_FFN = {"ReLU²": "relu2", "SwiGLU": "swiglu"}


def _positive(*values):
    return all(isinstance(v, int) and v > 0 for v in values)


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
    # added by this build
    score_function: str = "softmax"
    activation: str = "relu2"
    expert_dtype: str = "bf16"
    shared_experts: int = 1
    shared_expert_width: int | None = None
    allow_any_expert_width: bool = False

    def __post_init__(self):
        fill = dict(expert_width=self.width // 4 if isinstance(self.width, int) else None,
                    unique_layers=self.layers)
        for name, value in fill.items():
            if getattr(self, name) is None:
                object.__setattr__(self, name, value)
        if self.shared_expert_width is None:
            object.__setattr__(self, "shared_expert_width", self.expert_width)
        problems = [*self._shape_problems(), *self._routing_problems(),
                    *self._numeric_problems(), *self._build_problems()]
        if problems:
            raise ValueError("invalid MoE recipe: " + "; ".join(problems))

    # -- validation, grouped by what each check protects --------------------------------------

    def _shape_problems(self):
        if self.family not in EXPERT_FAMILIES:
            yield f"family {self.family!r} has no routed experts (expected one of {EXPERT_FAMILIES})"
        if not _positive(self.layers, self.width, self.heads, self.vocab_size, self.sequence_len,
                         self.routed_experts, self.expert_width, self.global_batch_tokens,
                         self.training_flops, self.loops):
            yield "sizes, budgets and loops must be positive integers"
            return
        if self.layers < 2:
            yield "an MoE stack needs at least two layers (the first stays dense)"
        if not 2 <= self.unique_layers <= self.layers:
            yield "stored (unique) layers must lie between two and the executed depth"
        if self.width < 24 or self.width % 4 or self.width % self.heads:
            yield "width must be at least 24 and divisible by four and by the head count"
        elif (self.width // self.heads) % 2:
            yield "the head dimension must be even"
        if self.expert_width != self.width // 4 and not self.allow_any_expert_width:
            yield (f"expert_width {self.expert_width} is not width // 4 = {self.width // 4} "
                   "(set allow_any_expert_width=True to allow it)")
        if self.global_batch_tokens % self.sequence_len:
            yield "global_batch_tokens must be a whole number of sequences"

    def _routing_problems(self):
        if not (isinstance(self.top_k, int) and isinstance(self.routed_experts, int)
                and 1 <= self.top_k <= self.routed_experts):
            yield f"top_k must lie in [1, routed_experts]; got {self.top_k}"
        if self.score_function not in SCORE_FUNCTIONS:
            yield f"score_function must be one of {SCORE_FUNCTIONS}"

    def _numeric_problems(self):
        for name in ("aux_loss_coeff", "z_loss_coeff"):
            v = getattr(self, name)
            if not (math.isfinite(v) and v >= 0):
                yield f"{name} must be a finite, non-negative coefficient"
        if not (math.isfinite(self.router_init_std) and self.router_init_std > 0):
            yield "router_init_std (the router's initial standard deviation) must be positive"

    def _build_problems(self):
        if self.activation not in ACTIVATIONS:
            yield f"activation must be one of {ACTIVATIONS}"
        if self.expert_dtype not in EXPERT_DTYPES:
            yield f"expert_dtype must be one of {EXPERT_DTYPES}"
        if self.shared_experts not in (0, 1):
            yield "shared_experts must be 0 or 1"
        if not _positive(self.shared_expert_width):
            yield "shared_expert_width must be a positive integer"

    # -- sizes ------------------------------------------------------------------------------

    @property
    def fc1_rows(self):
        """Rows of an expert's fc1: 2H for SwiGLU (gate, value), H for ReLU^2."""
        return 2 * self.expert_width if self.activation == "swiglu" else self.expert_width

    def expert_params(self, width=None):
        """Parameters of one expert of hidden width `width` (default expert_width): fc1 + fc2."""
        hidden = self.expert_width if width is None else width
        matrices = 3 if self.activation == "swiglu" else 2
        return matrices * self.width * hidden

    def moe_layer_params(self):
        """Parameters of one MoE layer as nexttransformer_amd.moe.MoELayer holds them."""
        return (self.routed_experts * self.expert_params() + self._shared_params()
                + self.width * self.routed_experts)

    def _shared_params(self):
        return self.shared_experts * self.expert_params(self.shared_expert_width)

    def counts(self):
        """Parameter counts of the whole model the scaling adapter builds: full MHA in every
        layer, a dense 4d ReLU^2 FFN in the first, an MoE layer in each of the others, the
        embedding and head over the vocabulary padded to 64, and the backbone's scalars.
        block_active counts what one token uses: top_k routed experts instead of all of them.
        Only defined for a flat stack of full-attention layers."""
        if self.family not in MHA_FAMILIES or self.unique_layers != self.layers:
            raise ValueError(f"parameter counts describe a flat full-attention stack; family "
                             f"{self.family!r} with {self.unique_layers} stored of {self.layers} "
                             "executed layers is not one")
        d = self.width
        per_layer_attention = 4 * d * d
        dense_first = 2 * d * (4 * d)
        router = d * self.routed_experts
        moe_stored = self.routed_experts * self.expert_params() + self._shared_params() + router
        moe_used = self.top_k * self.expert_params() + self._shared_params() + router
        blocks = self.layers * per_layer_attention + dense_first
        block_total = blocks + (self.layers - 1) * moe_stored
        block_active = blocks + (self.layers - 1) * moe_used
        vocab_rows = -(-self.vocab_size // 64) * 64
        io = 2 * d * vocab_rows
        scalars = _BACKBONE_SCALARS_PER_LAYER * self.layers + _BACKBONE_SCALARS_FIXED
        return dict(block_total=block_total, block_active=block_active, embedding_and_head=io,
                    native_small_parameters=scalars, model_total=block_total + io + scalars)

    # -- conversion from the reference's recipe ---------------------------------------------

    @classmethod
    def from_any(cls, recipe):
        """This build's recipe for `recipe`: itself, or -- for the reference's MoERecipe or any
        object carrying its fields -- a recipe with those field values read by name and the
        build-only keys at their defaults (ReLU^2, softmax, bf16, one shared expert of the
        routed experts' width), which is exactly the reference's layer."""
        if isinstance(recipe, cls):
            return recipe
        added = {"score_function", "activation", "expert_dtype", "shared_experts",
                 "shared_expert_width", "allow_any_expert_width"}
        names = [f.name for f in fields(cls) if f.name not in added]
        missing = [n for n in names if not hasattr(recipe, n)]
        if missing:
            raise ValueError(f"not an MoE recipe: {type(recipe).__name__} lacks {missing}")
        return cls(**{n: getattr(recipe, n) for n in names})


def load_t3_recipe(cell_id="moe-T3-L20", path=None):
    """The recipe of one expert cell of a T3 scaling manifest (the JSON the reference keeps at
    configs/scaling/t3.json; this package ships none, so `path` is required).

    The cell gives the depth, width, heads and expert width; its family's recipe gives the
    routed / selected / shared expert counts and the FFN activation, which are read, not
    assumed, and must be ones this build runs. Looped families store pre + core + post layers
    and execute the core `loops` times."""
    if path is None:
        raise ValueError("load_t3_recipe needs the path of a T3 scaling manifest")
    data = json.loads(Path(path).read_text())
    cells = {c["id"]: c for c in data["cells"] if c.get("family") in EXPERT_FAMILIES}
    if cell_id not in cells:
        raise ValueError(f"{cell_id!r} is not an expert-family cell of {path}")
    cell = cells[cell_id]
    family = next(f["recipe"] for f in data["families"] if f["id"] == cell["family"])
    if family.get("ffn") not in _MANIFEST_FFN:
        raise ValueError(f"family {cell['family']!r}: expert FFN {family.get('ffn')!r} is not "
                         f"one of {tuple(_MANIFEST_FFN)}")
    if not family.get("firstLayerDense", False):
        raise ValueError(f"family {cell['family']!r}: the scaling adapter keeps layer 0 dense")
    loops = family.get("loops", 1)
    stored = (cell["preLayers"] + cell["coreLayers"] + cell["postLayers"] if loops > 1
              else cell["layers"])
    return MoERecipe(layers=cell["layers"], width=cell["width"], heads=cell["heads"],
                     vocab_size=data["vocabSize"], sequence_len=data["sequenceLength"],
                     seed=data["seed"], global_batch_tokens=data["globalBatchTokens"],
                     training_flops=data["trainingFlops"], expert_width=cell["expertWidth"],
                     routed_experts=family["routedExperts"], top_k=family["selectedExperts"],
                     shared_experts=family["sharedExperts"],
                     activation=_MANIFEST_FFN[family["ffn"]], cell_id=cell_id,
                     family=cell["family"], unique_layers=stored, loops=loops)
