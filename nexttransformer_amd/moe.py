"""The MoE layer module over the HIP kernels: a drop-in for the reference's MoE engine.

Reference contract (nexttransformer/scaling/megatron_moe.py):
  * constructor (recipe, layer_number, pg_collection)                         :124-135
  * submodules router.weight [E, d]; experts.local_experts.{i}.linear_fc1/2;
    shared_experts.linear_fc1/2 (fp32 masters, bias-free)                      :58-78, 128-134
  * initialisation keyed by global expert id, fork_rng-style private seeds     :105-120, :27-29
  * last_load = per-expert token counts                                        :143, 149
  * MegatronFFN(recipe, layer_number, *, pg_collection, cpu_math) wraps the
    engine and returns only the output for a [B, S, d] hidden                  :153-182
  * build_model(recipe, *, pg_collection, cpu_math): MoE FFNs on every block but the dense
    first one, model.moe_recipe / model.moe_cpu_math set                       :185-208
The engine's forward here returns (out, aux_loss) rather than MCore's (out, bias=None); the
aux loss is the load-balance + z-loss of megatron_moe.py:44-45 in closed form. How its gradient
reaches the router is the engine's `aux_grad` mode:
  * "inject" (default; the reference engine's MCore semantics, megatron_moe.py:233-236): the
    backward adds d(aux)/d(router) scaled by the value last given to set_aux_loss_scale(),
    whether or not the caller's loss uses aux_loss, which is returned detached (a value to
    log). Only in training mode (module.train()), as MCore's router applies it.
  * "loss": aux_loss carries the graph and the caller adds it to its loss; the ffn plugin runs
    its engine this way because the plugin shell sums every `last_aux` tensor into the
    training loss (nexttransformer/models/plugins.py:24-25, lm.py:386-388).
The engine keeps its aux as `last_aux_loss`, never as `last_aux`, so the shell's sum over
modules counts it once, through the plugin block that owns the engine.

Compute: x is cast to bf16 (the reference's MasterLinear runs matmuls in the activation dtype,
megatron_moe.py:74-75); the router GEMM runs in fp32 on the bf16 values; expert GEMMs run on
bf16 copies of the fp32 masters (or, with expert_dtype "fp8", on e4m3 copies with 128 x 128
block scales and per-row quantised activations), repacked into [E, rows, cols] stacks only when
a master changes (tracked by the tensors' version counters, which in-place optimizer updates
bump).

Under autograd the layer runs its training path (_MoETrain: the forward keeps what the HIP
backward reads, and the gradients reach hidden and every fp32 master) for bf16 experts of any
width (widths that are not multiples of 64 run zero-padded); fp8 experts raise RuntimeError there
instead of returning a result without a graph. There is no CPU path.

Expert weight gradients (the `expert_grad` mode): with "accumulate" (the default) the backward
adds the routed experts' gradients into their .grad itself, whatever the caller asked autograd
for -- also under torch.autograd.grad(out, hidden) or loss.backward(inputs=[hidden]) -- and
per-parameter gradient hooks do not fire for them; this saves autograd's per-tensor work (about
a millisecond per backward at 256 experts). With "autograd" the expert masters are ordinary
inputs of the layer's autograd function: torch.autograd.grad can name them, `inputs=` is
honoured and hooks fire.

Weight caches: the bf16 / packed / fp8 operands are rebuilt when a master's address or version
counter changes. An update that does not bump the counter (a write through .data, or into the
storage from outside PyTorch) must be followed by invalidate_weights().
"""
import math

import torch
from torch import nn

from nexttransformer_amd import _native as nat
from nexttransformer_amd import ops
from nexttransformer_amd.moe_recipe import MoERecipe

SEED_LAYER_STRIDE = 100003  # megatron_moe.py:113-120: seed + 100003 * layer_number + index
AUX_GRAD_MODES = ("inject", "loss")
EXPERT_GRAD_MODES = ("accumulate", "autograd")

# Scale of the injected aux-loss gradient (MCore's MoEAuxLossAutoScaler main-loss scale), set by
# set_aux_loss_scale() before backward and read when the backward runs.
_aux_loss_scale = None


def set_aux_loss_scale(scale, *, device="cpu"):
    """Scale of the aux / z-loss gradient that "inject" engines add in their backward; call it
    before backward with the same 1/accumulation factor the main loss uses
    (megatron_moe.py:233-236). Stays in force until the next call; 1.0 until the first."""
    global _aux_loss_scale
    _aux_loss_scale = torch.tensor(float(scale), dtype=torch.float32, device=device)


_injected_cache = {}  # device -> (the scale tensor it was made from, its version, gradient)


def _injected_aux_grad(device):
    """{lb + z, lb, z} gradient [3] on `device` that an "inject" backward adds: (scale, 0, 0).
    Made once per device while the scale set by set_aux_loss_scale stays the same unmodified
    tensor (two small kernels less per backward); callers must not modify it."""
    s = _aux_loss_scale
    ver = None if s is None else s._version
    hit = _injected_cache.get(device)
    if hit is not None and hit[0] is s and hit[1] == ver:
        return hit[2]
    g = torch.zeros(3, device=device, dtype=torch.float32)
    if s is None:
        g[0] = 1.0
    else:
        g[0] = s.to(device, non_blocking=True)
    _injected_cache[device] = (s, ver, g)
    return g


_SCORE = {"softmax": nat.SCORE_SOFTMAX, "sigmoid": nat.SCORE_SIGMOID}
_ACT = {"swiglu": nat.ACT_SWIGLU, "relu2": nat.ACT_RELU2}


def input_init_(weight, generator=None):
    """U(-b, b), b = 0.4 * sqrt(3 / fan_in) (megatron_moe.py:27-29)."""
    bound = 0.4 * math.sqrt(3 / weight.shape[-1])
    return nn.init.uniform_(weight, -bound, bound, generator=generator)


def _round_up(n, m):
    return (n + m - 1) // m * m


def _seeded(seed):
    return torch.Generator(device="cpu").manual_seed(seed)


class Router(nn.Module):
    """The gating matrix: router.weight [E, d], fp32 (router dtype fp32, megatron_moe.py:42)."""

    def __init__(self, experts, width, device):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(experts, width, device=device, dtype=torch.float32))


class ExpertMLP(nn.Module):
    """One expert: linear_fc1 [rows, d], linear_fc2 [d, hidden], bias-free fp32 masters.

    rows = 2 * hidden for SwiGLU (rows [0, hidden) gate, [hidden, 2 hidden) value), hidden for
    the reference's ReLU^2 expert (megatron_moe.py:23-24, 51).
    """

    def __init__(self, width, hidden, gated, device):
        super().__init__()
        rows = 2 * hidden if gated else hidden
        self.linear_fc1 = nn.utils.skip_init(nn.Linear, width, rows, bias=False, device=device)
        self.linear_fc2 = nn.utils.skip_init(nn.Linear, hidden, width, bias=False, device=device)


class LocalExperts(nn.Module):
    """experts.local_experts.{i}: every routed expert (one GPU, so local ids are global ids)."""

    def __init__(self, count, width, hidden, gated, device):
        super().__init__()
        self.local_experts = nn.ModuleList(
            ExpertMLP(width, hidden, gated, device) for _ in range(count))


def _pool_masters(linears):
    """Puts the fp32 weights of same-shaped linears into one contiguous [n, rows, cols] buffer
    and makes each linear's weight a Parameter on its slice (same names, shapes and values), so
    the stack of them needs no copy; returns the buffer."""
    w0 = linears[0].weight
    pool = torch.empty((len(linears),) + tuple(w0.shape), device=w0.device, dtype=w0.dtype)
    for i, lin in enumerate(linears):
        pool[i].copy_(lin.weight.detach())
        lin.weight = nn.Parameter(pool[i], requires_grad=lin.weight.requires_grad)
    return pool


def _stacked(pool, weights):
    """[n, rows, cols] fp32 of the weights: the pool itself when every weight still sits on its
    slice of it (in-place updates keep that; replacing a weight's tensor, or moving the module
    to another device, does not), else a stacked copy."""
    if pool is not None and pool.device == weights[0].device:
        base, step = pool.data_ptr(), pool.stride(0) * pool.element_size()
        if all(w.data_ptr() == base + i * step for i, w in enumerate(weights)):
            return pool
    return torch.stack([w.detach() for w in weights])


def _ep_size(pg_collection):
    ep = getattr(pg_collection, "ep", None)
    if ep is None:
        return 1
    size = ep.size() if callable(getattr(ep, "size", None)) else getattr(ep, "size", 1)
    return int(size)


class _MoETrain(torch.autograd.Function):
    """The layer with gradients (bf16 experts): ops.moe_forward, then ops.moe_backward. Its
    inputs after x are router.weight and the shared expert's fp32 masters, so autograd hands
    each its own gradient; the bf16 operands the kernels read are the layer's cached copies of
    the masters (MasterLinear casts its master per call, megatron_moe.py:58-78; the cache is
    rebuilt when a master changes). With expert_grad "accumulate" (the default) the routed
    experts' masters (two per expert) are not inputs: autograd's per-input bookkeeping costs a
    few microseconds per tensor (over a millisecond per step at 256 experts), so the backward
    adds their gradients to .grad itself, from one fp32 stack per projection
    (MoELayer._accumulate_expert_grads); with "autograd" they are inputs like the others.
    `anchor`, an empty tensor that requires grad, keeps the backward in the graph when nothing
    else does. x and the weights may be zero-padded to widths the kernels take (MoELayer.
    packed_weights); the gradients handed back have the masters' shapes."""

    @staticmethod
    def forward(ctx, x, cfg, anchor, *masters):
        layer = cfg["layer"]
        w = layer.packed_weights(keep_plain=True)
        out, aux, state = ops.moe_forward(
            x, w["router_t"], w["w1"], w["w2"], top_k=cfg["top_k"], score_fn=cfg["score_fn"],
            activation=cfg["activation"], aux_coeff=cfg["aux_coeff"], z_coeff=cfg["z_coeff"],
            logit_bias=layer.logit_bias, shared_w1=w["shared_w1"], shared_w2=w["shared_w2"],
            want_logits=True, packed=w["packed"], keep=True)
        cfg["counts"] = state["counts"]
        ctx.cfg, ctx.state, ctx.x, ctx.w = cfg, state, x, w
        # an output the loss does not use gets None, not a zero-filled gradient
        ctx.set_materialize_grads(False)
        return out, aux

    @staticmethod
    def backward(ctx, grad_out, grad_aux):
        cfg, x, w = ctx.cfg, ctx.x, ctx.w
        layer = cfg["layer"]
        bw = layer.backward_weights(w)
        if cfg["inject"]:  # MCore: the aux gradient arrives whatever the caller's loss holds
            injected = _injected_aux_grad(x.device)
            grad_aux = injected if grad_aux is None else grad_aux + injected
        if grad_out is None:
            grad_out = torch.zeros(x.shape, device=x.device, dtype=torch.bfloat16)
        g = ops.moe_backward(grad_out, None if grad_aux is None else grad_aux.contiguous(), x,
                             w["router_t"], bw, ctx.state, top_k=cfg["top_k"],
                             score_fn=cfg["score_fn"], activation=cfg["activation"],
                             aux_coeff=cfg["aux_coeff"], z_coeff=cfg["z_coeff"],
                             weight_grads_fp32=True)
        ctx.state = ctx.x = ctx.w = None
        g = layer._unpadded_grads(g)
        grads = [g["x"], None, None, g["router"]]
        if cfg["expert_autograd"]:  # fc1, fc2 of expert 0, then expert 1, ... as inputs
            for a, b in zip(g["w1"].unbind(0), g["w2"].unbind(0)):
                grads += [a, b]
        else:
            pooled = layer._masters(pooled_only=True)  # fc1, fc2 of expert 0, then expert 1, ...
            layer._accumulate_expert_grads(pooled[0::2], g["w1"])
            layer._accumulate_expert_grads(pooled[1::2], g["w2"])
        if g["shared_w1"] is not None:
            grads += [g["shared_w1"][0], g["shared_w2"][0]]
        return tuple(grads)


class MoELayer(nn.Module):
    """MoE layer forward on one MI355X: router -> route plan -> grouped GEMMs -> combine + aux.

    forward(hidden [..., d]) -> (out [..., d] in hidden's dtype, aux_loss fp32 scalar).
    """

    def __init__(self, recipe, layer_number: int, pg_collection=None, *, device=None,
                 aux_grad="inject", expert_grad="accumulate"):
        super().__init__()
        recipe = MoERecipe.from_any(recipe)
        if aux_grad not in AUX_GRAD_MODES:
            raise ValueError(f"aux_grad must be one of {AUX_GRAD_MODES}")
        if expert_grad not in EXPERT_GRAD_MODES:
            raise ValueError(f"expert_grad must be one of {EXPERT_GRAD_MODES}")
        if layer_number < 1:
            raise ValueError("layer_number counts from one")
        if _ep_size(pg_collection) != 1:
            raise ValueError("this build runs the MoE layer on one GPU; expert parallelism "
                             "(pg_collection.ep size > 1) is not supported")
        if recipe.routed_experts > nat.MAX_EXPERTS or recipe.top_k > nat.MAX_TOPK:
            raise ValueError(f"the HIP router supports at most {nat.MAX_EXPERTS} experts and "
                             f"top-{nat.MAX_TOPK}")
        if device is None:
            device = (torch.device("cuda", torch.cuda.current_device())
                      if torch.cuda.is_available() else torch.device("cpu"))
        self.recipe = recipe
        self.layer_number = layer_number
        self.aux_grad = aux_grad
        self.expert_grad = expert_grad
        gated = recipe.activation == "swiglu"
        self.router = Router(recipe.routed_experts, recipe.width, device)
        self.experts = LocalExperts(recipe.routed_experts, recipe.width, recipe.expert_width,
                                    gated, device)
        experts = list(self.experts.local_experts)
        self._fc1_pool = _pool_masters([e.linear_fc1 for e in experts])
        self._fc2_pool = _pool_masters([e.linear_fc2 for e in experts])
        self._pool_ptrs = None  # the pooled weights' addresses on their pool slices
        self._pools_placed = False  # every pooled weight on its slice (set by _masters_key)
        self._param_tables = None
        self.shared_experts = (ExpertMLP(recipe.width, recipe.shared_expert_width, gated, device)
                               if recipe.shared_experts else None)
        # Optional fixed per-expert logit bias [E] fp32 added after the gating GEMM (not a
        # parameter; None = no bias, the reference router): used to impose a routing skew.
        self.register_buffer("logit_bias", None)
        self._last_counts = None
        self.last_aux_loss = None
        self.last_aux_parts = None
        self._pack_key = None
        self._packed = None
        self.reset_parameters()

    @property
    def last_load(self):
        """Per-expert token counts of the last forward, int64 [E] (None before the first): the
        kernels' int32 counts, converted on first access rather than in every forward."""
        c = self._last_counts
        if c is not None and c.dtype != torch.int64:
            c = self._last_counts = c.to(torch.int64)
        return c

    # -- initialisation --------------------------------------------------------------------

    @torch.no_grad()
    def reset_parameters(self):
        """Initialise as megatron_moe.py:105-120 does on its CPU path: every expert draws from
        its own CPU generator seeded seed + 100003 * layer + global expert id; the shared expert
        uses id E and the router id E + 1. fc1 ~ U(+-0.4 sqrt(3/d)), fc2 = 0, router ~ N(0, std).
        Values are drawn on the CPU and copied, so they are identical on every device."""
        r = self.recipe
        base = r.seed + SEED_LAYER_STRIDE * self.layer_number

        def init_expert(expert, seed):
            fc1 = torch.empty(expert.linear_fc1.weight.shape, dtype=torch.float32, device="cpu")
            input_init_(fc1, _seeded(seed))
            expert.linear_fc1.weight.copy_(fc1)
            expert.linear_fc2.weight.zero_()

        for i, expert in enumerate(self.experts.local_experts):
            init_expert(expert, base + i)
        if self.shared_experts is not None:
            init_expert(self.shared_experts, base + r.routed_experts)
        w = torch.empty(self.router.weight.shape, dtype=torch.float32, device="cpu")
        nn.init.normal_(w, std=r.router_init_std, generator=_seeded(base + r.routed_experts + 1))
        self.router.weight.copy_(w)
        self.invalidate_weights()

    def invalidate_weights(self):
        """Drops the cached kernel operands (bf16 / packed / fp8 copies of the masters and the
        backward's transposes), so the next forward rebuilds them from the masters. The cache
        follows each master's address and version counter, which in-place updates bump
        (torch.optim steps, copy_ / add_ under no_grad); an update that bypasses the counter
        (writes through .data, or into the storage from outside PyTorch) must call this."""
        self._pack_key = None
        self._packed = None

    # -- expert weight gradients -----------------------------------------------------------

    def _accumulate_expert_grads(self, params, grad):
        """Adds one projection's expert gradients, the fp32 stack grad [E, rows, cols], into the
        experts' .grad as autograd would (a .grad that is None takes the gradient, one that is
        set accumulates it; parameters that do not require grad are skipped). When no .grad is
        set (zero_grad with set_to_none), each takes its slice of `grad`; when every .grad is
        still its slice of one such stack (same storage, consecutive, contiguous), the new
        gradients are added to that stack in one pass; otherwise tensor by tensor."""
        if all(p.grad is None for p in params):
            for p, v in zip(params, grad.unbind(0)):
                if p.requires_grad:
                    p.grad = v
            return
        g0 = params[0].grad
        if (g0 is not None and g0.dtype == grad.dtype and g0.device == grad.device
                and tuple(g0.shape) == tuple(grad.shape[1:]) and g0.is_contiguous()):
            storage, base, step = g0.untyped_storage().data_ptr(), g0.data_ptr(), g0.nbytes
            if all(p.grad is not None and p.grad.is_contiguous()
                   and p.grad.data_ptr() == base + i * step
                   and p.grad.untyped_storage().data_ptr() == storage
                   for i, p in enumerate(params)):
                # as_strided checks that the extent lies inside the storage
                g0.as_strided(grad.shape, (g0.numel(),) + tuple(g0.stride()),
                              g0.storage_offset()).add_(grad)
                return
        for p, v in zip(params, grad.unbind(0)):
            if not p.requires_grad:
                continue
            if p.grad is None:
                p.grad = v
            else:
                p.grad.add_(v)

    # -- packed bf16 weights ---------------------------------------------------------------

    def _masters(self, pooled_only=False, skip_pooled=False):
        """router.weight, each expert's fc1 and fc2 weights, then the shared expert's (read from
        the modules' parameter tables, which a replaced weight updates in place); only the
        experts' with pooled_only, all but theirs with skip_pooled."""
        if self._param_tables is None:
            lins = []
            for e in self.experts.local_experts:
                lins += [e.linear_fc1, e.linear_fc2]
            shared = ([] if self.shared_experts is None else
                      [self.shared_experts.linear_fc1, self.shared_experts.linear_fc2])
            self._param_tables = ([self.router._parameters],
                                  [lin._parameters for lin in lins],
                                  [lin._parameters for lin in shared])
        router, pooled, shared = self._param_tables
        if pooled_only:
            return [t["weight"] for t in pooled]
        if skip_pooled:
            return [t["weight"] for t in router + shared]
        return [t["weight"] for t in router + pooled + shared]

    def _masters_key(self):
        """Identifies the current values of every master: the tensors' addresses and version
        counters. The pooled expert weights share their pool's version counter (an in-place
        update of any of them bumps it), so while they all sit on their pool slices one
        version stands for each pool."""
        masters = self._masters()
        ptrs = tuple(p.data_ptr() for p in masters)
        pools = (self._fc1_pool, self._fc2_pool)
        if self._pool_ptrs is None and pools[0] is not None:
            # expert i's fc1 and fc2 weights on slice i of their pools (the masters' order)
            (b1, b2), (s1, s2) = ((p.data_ptr() for p in pools),
                                  (p.stride(0) * p.element_size() for p in pools))
            self._pool_ptrs = tuple(x for i in range(pools[0].shape[0])
                                    for x in (b1 + i * s1, b2 + i * s2))
        self._pools_placed = (self._pool_ptrs is not None
                              and ptrs[1:1 + len(self._pool_ptrs)] == self._pool_ptrs
                              and pools[0].device == masters[1].device)
        if self._pools_placed:
            n = 1 + len(self._pool_ptrs)
            return (ptrs, masters[0]._version, pools[0]._version, pools[1]._version,
                    tuple(p._version for p in masters[n:]))
        return ptrs, tuple(p._version for p in masters)

    @torch.no_grad()
    def backward_weights(self, w):
        """The backward's GEMM operands for the weights `w` (packed_weights(keep_plain=True))
        a forward used, kept in `w` itself, so a backward always uses operands built from its
        own forward's weights (each operand on first use)."""
        if "_bw" not in w:
            w["_bw"] = ops.backward_weights(w["w1_plain"], w["w2_plain"], w["shared_w1_plain"],
                                            w["shared_w2_plain"], w["router_t"],
                                            w1_t=w["w1_t"], w2_t=w["w2_t"],
                                            shared_w2_t=w["shared_w2_t"],
                                            w1_t_packed=w["w1_t_packed"],
                                            w2_t_packed=w["w2_t_packed"],
                                            shared_w2_t_packed=w["shared_w2_t_packed"],
                                            first=w.get("first"))
        return w["_bw"]

    def _unpadded_grads(self, g):
        """moe_backward's gradients of the zero-padded operands (x [T, dp], router [E, dp],
        fc1 [E, (2) Hp, dp], fc2 [E, dp, Hp], the shared expert's likewise) cut back to the
        masters' shapes: the padding entries are constants, so the masters' gradients are the
        padded gradients' entries at the masters' positions (for SwiGLU, fc1's value half starts
        at row Hp)."""
        r = self.recipe
        d = r.width
        gated = r.activation == "swiglu"

        def fc1(t, hidden):
            hp = t.shape[1] // (2 if gated else 1)
            if hp == hidden and t.shape[2] == d:
                return t
            if gated:
                return torch.cat([t[:, :hidden, :d], t[:, hp:hp + hidden, :d]], 1)
            return t[:, :hidden, :d].contiguous()

        def fc2(t, hidden):
            return t if tuple(t.shape[1:]) == (d, hidden) else t[:, :d, :hidden].contiguous()

        out = dict(g)
        if g["router"].shape[1] != d:
            out["router"] = g["router"][:, :d].contiguous()
        out["w1"], out["w2"] = fc1(g["w1"], r.expert_width), fc2(g["w2"], r.expert_width)
        if g["shared_w1"] is not None:
            out["shared_w1"] = fc1(g["shared_w1"], r.shared_expert_width)
            out["shared_w2"] = fc2(g["shared_w2"], r.shared_expert_width)
        return out

    @torch.no_grad()
    def packed_weights(self, keep_plain=False):
        """Device weights the kernels read, rebuilt only when a master tensor changed:
        router_t fp32 [dp, E]; w1 [E, rows, dp]; w2 [E, dp, Hp]; shared_w1/2 [1, ...];
        bf16 (the up projections' w1 in the packed fragment order of pack_expert_weights when
        `packed`[0], the down projections' w2 when `packed`[1]), or for expert_dtype "fp8" e4m3
        codes (uint8, always packed: `packed` True) with their 128 x 128 block scales (w1_scale,
        w2_scale, shared_w1_scale, shared_w2_scale).

        The bf16 GEMM tiles K and the SwiGLU halves in multiples of 64, the fp8 GEMM's scale
        blocks are 128 wide, so d and the expert widths are zero-padded up to dp, Hp when they
        are not already multiples: zero input features add exact zeros to every dot product, and
        a zero hidden unit has act(0) = 0 under both SwiGLU and ReLU^2, so the padded layer
        computes the same values (an all-zero fp8 block gets scale 1 and codes 0).
        """
        key = self._masters_key()
        if key != self._pack_key or (keep_plain and "w1_plain" not in self._packed):
            r = self.recipe
            fp8 = r.expert_dtype == "fp8"
            align = 128 if fp8 else 64
            dp = _round_up(r.width, align)
            gated = r.activation == "swiglu"
            dtype = torch.float32 if fp8 else torch.bfloat16
            # The packed-weight GEMM (fragment-ordered weights streamed into registers) for a
            # projection when its K and width qualify for every expert kind (routed, shared) and
            # the weights live on the GPU; fp8 always. (The T3 cell: both projections packed,
            # the down projection's K = 320 on the kernel's odd K-step path.)
            widths = [r.expert_width] + ([r.shared_expert_width] if self.shared_experts else [])
            on_gpu = self.router.weight.is_cuda
            # Training (keep_plain) rebuilds these after every update. Where the conversion
            # pass writes the packed layout itself (bf16, no padding, on the GPU) packing costs
            # nothing extra; elsewhere it is a second pass, worth it only for even K-step counts.
            fused = (not fp8 and on_gpu and dp == r.width
                     and all(_round_up(h, align) == h for h in widths))
            extra_pass = keep_plain and not fused
            pk_up = fp8 or (on_gpu and all(ops.prefers_packed(
                dp, _round_up(h, align), nat.EPI_SWIGLU if gated else nat.EPI_RELU2,
                repacked_each_step=extra_pass) for h in widths))
            pk_down = fp8 or (on_gpu and all(
                ops.prefers_packed(_round_up(h, align), dp, nat.EPI_NONE,
                                   repacked_each_step=extra_pass) for h in widths))

            def stack(experts, hidden, pools=(None, None), need_w1=False):
                hp = _round_up(hidden, align)
                if not fp8 and hp == hidden and dp == r.width and self.router.weight.is_cuda:
                    # one pass over each fp32 master stack writes what the kernels read: the
                    # packed or plain weights and, for the backward, the transposes (packed
                    # when their dgrad projection takes the packed GEMM)
                    up = nat.EPI_SWIGLU if gated else nat.EPI_RELU2
                    rows1 = (2 if gated else 1) * hidden
                    t1 = keep_plain and ops.prefers_packed(rows1, r.width, nat.EPI_NONE,
                                                           repacked_each_step=False)
                    t2 = keep_plain and ops.prefers_packed(r.width, hidden, nat.EPI_NONE,
                                                           repacked_each_step=False)
                    # the pools themselves when the key found every weight on its slice (no
                    # per-expert attribute walk: at 256 experts that costs 0.4 ms of host time)
                    placed = pools[0] is not None and self._pools_placed
                    src1 = pools[0] if placed else _stacked(
                        pools[0], [e.linear_fc1.weight for e in experts])
                    src2 = pools[1] if placed else _stacked(
                        pools[1], [e.linear_fc2.weight for e in experts])
                    w1, w1t, w1p, w1tp = ops.convert_pack_expert_weights.raw(
                        src1, up, not pk_up or need_w1, keep_plain and not t1, pk_up, t1)
                    w2, w2t, w2p, w2tp = ops.convert_pack_expert_weights.raw(
                        src2, nat.EPI_NONE, not pk_down, keep_plain and not t2, pk_down, t2)
                    some = lambda t: t if t.numel() else None
                    plain.append((some(w1), some(w2), some(w1t), some(w2t), some(w1tp),
                                  some(w2tp)))
                    return (w1p if pk_up else w1, None, w2p if pk_down else w2, None)
                if hp == hidden and dp == r.width:
                    w1 = torch.stack([e.linear_fc1.weight.detach() for e in experts]).to(dtype)
                    w2 = torch.stack([e.linear_fc2.weight.detach() for e in experts]).to(dtype)
                else:
                    n = len(experts)
                    dev = experts[0].linear_fc1.weight.device
                    w1 = torch.zeros(n, (2 if gated else 1) * hp, dp, device=dev, dtype=dtype)
                    w2 = torch.zeros(n, dp, hp, device=dev, dtype=dtype)
                    for i, e in enumerate(experts):
                        fc1 = e.linear_fc1.weight.detach()
                        if gated:
                            w1[i, :hidden, :r.width] = fc1[:hidden]
                            w1[i, hp:hp + hidden, :r.width] = fc1[hidden:]
                        else:
                            w1[i, :hidden, :r.width] = fc1
                        w2[i, :r.width, :hidden] = e.linear_fc2.weight.detach()
                if not fp8:
                    up = nat.EPI_SWIGLU if gated else nat.EPI_RELU2
                    w1, w2 = w1.contiguous(), w2.contiguous()
                    plain.append((w1, w2, None, None, None, None))
                    return (ops.pack_expert_weights.raw(w1, up) if pk_up else w1, None,
                            ops.pack_expert_weights.raw(w2, nat.EPI_NONE) if pk_down else w2, None)
                w1q, w1s = ops.quantize_fp8_blockwise(w1.contiguous())
                w2q, w2s = ops.quantize_fp8_blockwise(w2.contiguous())
                up = nat.EPI_SWIGLU if gated else nat.EPI_RELU2
                return (ops.pack_expert_weights_fp8(w1q, up), w1s,
                        ops.pack_expert_weights_fp8(w2q, nat.EPI_NONE), w2s)

            plain = []  # the bf16 [E, rows, cols] stacks before packing (for the backward)
            packed = dict(shared_w1=None, shared_w2=None,
                          shared_w1_scale=None, shared_w2_scale=None,
                          packed=True if fp8 else (pk_up, pk_down))
            (packed["w1"], packed["w1_scale"], packed["w2"],
             packed["w2_scale"]) = stack(list(self.experts.local_experts), r.expert_width,
                                         (self._fc1_pool, self._fc2_pool))
            if self.shared_experts is not None:
                (packed["shared_w1"], packed["shared_w1_scale"], packed["shared_w2"],
                 packed["shared_w2_scale"]) = stack([self.shared_experts], r.shared_expert_width,
                                                     need_w1=True)
            if keep_plain and not fp8:
                (packed["w1_plain"], packed["w2_plain"], packed["w1_t"], packed["w2_t"],
                 packed["w1_t_packed"], packed["w2_t_packed"]) = plain[0]
                (packed["shared_w1_plain"], packed["shared_w2_plain"], _, packed["shared_w2_t"],
                 _, packed["shared_w2_t_packed"]) = plain[1] if len(plain) > 1 else (None,) * 6
            # the router's operands after the expert conversions, whose GPU time then covers
            # this host work: w_router_t and, for the backward, the first operand in one kernel
            rw = self.router.weight.detach()
            packed["first"] = None
            if on_gpu:
                want_first = keep_plain and not fp8
                sw1 = packed.get("shared_w1_plain") if want_first else None
                if rw.dtype != torch.float32 or rw.stride(1) != 1:
                    rw = rw.float().contiguous()
                packed["router_t"], first = ops.router_operands.raw(
                    rw, dp, None if sw1 is None else sw1[0], want_first)
                if want_first:
                    packed["first"] = first
            else:
                router_t = torch.zeros(dp, r.routed_experts, device=rw.device,
                                       dtype=torch.float32)
                router_t[:r.width] = rw.t()
                packed["router_t"] = router_t
            self._packed = packed
            self._pack_key = key
        return self._packed

    # -- forward ---------------------------------------------------------------------------

    def forward(self, hidden):
        r = self.recipe
        if hidden.shape[-1] != r.width:
            raise ValueError(f"hidden width {hidden.shape[-1]} != recipe width {r.width}")
        if not hidden.is_cuda:
            raise ValueError("the MoE layer runs on the GPU only (no CPU path)")
        if self.router.weight.device != hidden.device:
            raise ValueError(f"parameters are on {self.router.weight.device}, hidden on "
                             f"{hidden.device}")
        if torch.is_grad_enabled() and (hidden.requires_grad or
                                        any(p.requires_grad for p in self.parameters())):
            return self._forward_train(hidden)
        w = self.packed_weights()
        x = hidden.reshape(-1, r.width)
        dp = w["router_t"].shape[0]
        if dp != r.width:
            xp = torch.zeros(x.shape[0], dp, device=x.device, dtype=torch.bfloat16)
            xp[:, :r.width] = x
            x = xp
        elif x.dtype != torch.bfloat16 or x.stride(-1) != 1:
            x = x.to(torch.bfloat16).contiguous()
        out, aux, state = ops.moe_forward(
            x, w["router_t"], w["w1"], w["w2"], top_k=r.top_k,
            score_fn=_SCORE[r.score_function], activation=_ACT[r.activation],
            aux_coeff=r.aux_loss_coeff, z_coeff=r.z_loss_coeff, logit_bias=self.logit_bias,
            shared_w1=w["shared_w1"], shared_w2=w["shared_w2"], w1_scale=w["w1_scale"],
            w2_scale=w["w2_scale"], shared_w1_scale=w["shared_w1_scale"],
            shared_w2_scale=w["shared_w2_scale"], packed=w["packed"])
        if dp != r.width:
            out = out[:, :r.width]
        self._last_counts = state["counts"]
        self.last_aux_parts = aux
        self.last_aux_loss = aux[0]
        out = out.reshape(hidden.shape).to(hidden.dtype)
        return out, self.last_aux_loss


    def _forward_train(self, hidden):
        """Forward with gradients to hidden and every master (bf16 experts). Widths that are not
        multiples of 64 (the reference's debug recipe: d = 32, expert width 8) run zero-padded,
        as the inference forward does; the gradients come back in the masters' shapes."""
        r = self.recipe
        if r.expert_dtype == "fp8":
            raise RuntimeError("the MoE backward covers bf16 experts; run fp8 experts under "
                               "torch.no_grad()")
        if not self.router.weight.is_cuda:
            raise ValueError("the MoE layer runs on the GPU only (no CPU path)")
        x = hidden.reshape(-1, r.width).to(torch.bfloat16)
        dp = _round_up(r.width, 64)
        if dp != r.width:
            x = nn.functional.pad(x, (0, dp - r.width))
        x = x.contiguous()
        inject = self.aux_grad == "inject"
        autograd_experts = self.expert_grad == "autograd"
        cfg = dict(layer=self, top_k=r.top_k, score_fn=_SCORE[r.score_function],
                   activation=_ACT[r.activation], aux_coeff=r.aux_loss_coeff,
                   z_coeff=r.z_loss_coeff, inject=inject and self.training,
                   expert_autograd=autograd_experts)
        anchor = torch.empty(0, device=x.device, requires_grad=True)
        masters = self._masters(skip_pooled=not autograd_experts)
        out, aux = _MoETrain.apply(x, cfg, anchor, *masters)
        if dp != r.width:
            out = out[:, :r.width]
        self._last_counts = cfg["counts"]
        self.last_aux_parts = aux.detach()
        # "inject": the gradient comes from the backward itself, so the returned value is
        # detached and adding it to a loss changes nothing
        self.last_aux_loss = aux[0].detach() if inject else aux[0]
        return out.reshape(hidden.shape).to(hidden.dtype), self.last_aux_loss


class MoEFFN(nn.Module):
    """The block-level wrapper (megatron_moe.py:153-182): forward(hidden [B, S, d]) -> [B, S, d].

    Accepts this build's MoERecipe or the reference's. Its engine injects the aux-loss gradient
    as MCore does (set_aux_loss_scale), so, like the reference's MegatronFFN, it exposes no
    `last_aux` for a trainer to add; the engine's last_aux_loss holds the value for logging.
    The engine's per-row computation and its aux loss (sums over all tokens) do not depend on
    the token order, so no [B, S] <-> [S, B] transpose is needed around it.
    """

    def __init__(self, recipe, layer_number, *, pg_collection=None, cpu_math=False, device=None):
        super().__init__()
        if cpu_math:
            raise ValueError("this build has no CPU math path: the MoE layer runs on the GPU")
        self.engine = MoELayer(recipe, layer_number, pg_collection, device=device,
                               aux_grad="inject")

    def forward(self, hidden):
        out, _ = self.engine(hidden)
        return out


MegatronFFN = MoEFFN


def install_moe_ffns(model, recipe, *, pg_collection=None, cpu_math=False, device=None):
    """Puts MoE FFNs into a native backbone the way the scaling adapter does
    (megatron_moe.py:203-207): block `index` > 0 of model.transformer.h gets
    MegatronFFN(recipe, layer_number=index + 1); block 0 keeps its dense FFN. Sets
    model.moe_recipe (the recipe object as given, so a reference recipe keeps its own counts()
    for the reference optimizer, megatron_optimizer.py:60-65) and model.moe_cpu_math."""
    if cpu_math:
        raise ValueError("this build has no CPU math path: the MoE layer runs on the GPU")
    blocks = list(model.transformer.h)
    if len(blocks) < 2:
        raise ValueError("the backbone needs at least two blocks (the first stays dense)")
    if device is None:
        device = next(model.parameters()).device
    for index, block in enumerate(blocks):
        if index > 0:
            block.mlp = MoEFFN(recipe, index + 1, pg_collection=pg_collection, device=device)
    model.moe_recipe = recipe
    model.moe_cpu_math = False
    return model


def build_model(recipe, *, pg_collection=None, cpu_math=False, backbone=None):
    """The scaling adapter's build_model (megatron_moe.py:185-208): the family's native backbone
    with MoE FFNs on every block but the dense first one.

    backbone(recipe, device) -> model builds the native backbone (an nn.Module whose
    model.transformer.h lists blocks with an `mlp`). By default it is NextTransformer's own
    builder, imported from the installed `nexttransformer` package, configured as the adapter
    configures it (megatron_moe.py:191-202); this package does not ship that backbone."""
    r = MoERecipe.from_any(recipe)
    if r.family not in ("moe", "looped"):
        raise ValueError(f"family {r.family!r} has no native full-attention backbone")
    if cpu_math:
        raise ValueError("this build has no CPU math path: the MoE layer runs on the GPU")
    device = torch.device("cuda", torch.cuda.current_device())
    model = (backbone or _native_backbone)(recipe, device)
    return install_moe_ffns(model, recipe, pg_collection=pg_collection, device=device)


def _native_backbone(recipe, device):
    """NextTransformer's native backbone for `recipe` (needs the nexttransformer package):
    full-MHA, no value embeddings, stored depth unique_layers and executed depth layers, a
    4 x width dense FFN, window pattern "L" (megatron_moe.py:191-202)."""
    from dataclasses import replace
    from nexttransformer.models.config import debug_config
    from nexttransformer.models.lm import build_model as native_build
    method = "fixed_recursive" if recipe.family == "looped" else "mha_no_ve"
    config = replace(debug_config(method, width=recipe.width, sequence_len=recipe.sequence_len),
                     layers=recipe.unique_layers, heads=recipe.heads, mlp_width=4 * recipe.width,
                     vocab_size=recipe.vocab_size, window_pattern="L")
    if config.n_layer != recipe.unique_layers or config.maximum_depth != recipe.layers:
        raise ValueError("the backbone's stored and executed depths differ from the recipe's")
    return native_build(config, device=f"cuda:{device.index}", seed=recipe.seed)
