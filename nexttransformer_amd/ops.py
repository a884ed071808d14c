"""torch.library custom ops ("ntmoe::*") over the C ABI of libnt_moe.so.

Each op checks devices, dtypes and shapes (ValueError, as the reference's config checks do,
nexttransformer/scaling/moe_recipe.py:54-72), allocates its outputs with torch's caching
allocator, and enqueues the HIP kernels on the current stream. Status codes from the library
become ValueError (bad arguments) or RuntimeError (launch failures). There is no CPU path: a
CPU tensor is a ValueError and a missing library raises NativeLibraryMissing.
"""
import ctypes
from typing import Optional

import torch
from torch import Tensor

from nexttransformer_amd import _native as nat
from nexttransformer_amd._native import ptr


def _stream(device):
    """The current HIP stream of `device` as a raw handle."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require(cond, message):
    if not cond:
        raise ValueError(message)


def _on_gpu(*tensors):
    for t in tensors:
        if t is not None:
            _require(t.is_cuda, f"ntmoe ops run on the GPU only; got a {t.device} tensor")


def _nblk(T):
    return (T + nat.ROUTE_BLOCK - 1) // nat.ROUTE_BLOCK


def _custom_op(name):
    """torch.library.custom_op(name) that keeps the undecorated function as `.raw`. The layer's
    own forward, backward and weight rebuild (moe_forward, moe_backward, Projection, the module)
    call `.raw`: the dispatcher's per-call host cost (about 20 us) is more than some of the
    kernels take, and with a dozen calls per training step it left the GPU waiting on the host."""
    def deco(fn):
        op = torch.library.custom_op(name, mutates_args=())(fn)
        op.raw = fn
        return op
    return deco


# ---------------------------------------------------------------------------------------------
# router

@_custom_op("ntmoe::router")
def router(x: Tensor, w_router_t: Tensor, bias: Optional[Tensor], k: int, score_fn: int,
           want_logits: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(logits [T,E] or empty, ids [T,k] int32, weights [T,k], prob_partial, z_partial)."""
    _on_gpu(x, w_router_t, bias)
    _require(x.dtype == torch.bfloat16 and x.dim() == 2, "router: x must be bf16 [T, d]")
    _require(x.stride(1) == 1, "router: x rows must be contiguous")
    _require(w_router_t.dtype == torch.float32 and w_router_t.is_contiguous(),
             "router: w_router_t must be contiguous fp32 [d, E]")
    T, d = x.shape
    _require(w_router_t.shape[0] == d, "router: w_router_t must be [d, E]")
    E = w_router_t.shape[1]
    if bias is not None:
        _require(bias.dtype == torch.float32 and bias.shape == (E,) and bias.is_contiguous(),
                 "router: bias must be contiguous fp32 [E]")
    dev = x.device
    logits = torch.empty((T, E) if want_logits else (0,), device=dev, dtype=torch.float32)
    ids = torch.empty(T, k, device=dev, dtype=torch.int32)
    w = torch.empty(T, k, device=dev, dtype=torch.float32)
    pp = torch.empty(_nblk(T), E, device=dev, dtype=torch.float32)
    zp = torch.empty(_nblk(T), device=dev, dtype=torch.float32)
    lib = nat.load()
    ws_bytes = lib.nt_moe_router_workspace_bytes(T, d, E, k)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    st = lib.nt_moe_router_fwd(ptr(x), x.stride(0), ptr(w_router_t), ptr(bias), T, d, E, k,
                               score_fn, ptr(logits) if want_logits else None, ptr(ids), ptr(w),
                               ptr(pp), ptr(zp), ptr(ws), ws_bytes, _stream(dev))
    nat.check(st, "ntmoe::router")
    return logits, ids, w, pp, zp


@router.register_fake
def _(x, w_router_t, bias, k, score_fn, want_logits):
    T, E = x.shape[0], w_router_t.shape[1]
    f = x.new_empty
    return (f((T, E) if want_logits else (0,), dtype=torch.float32),
            f((T, k), dtype=torch.int32), f((T, k), dtype=torch.float32),
            f((_nblk(T), E), dtype=torch.float32), f((_nblk(T),), dtype=torch.float32))


@_custom_op("ntmoe::topk_from_logits")
def topk_from_logits(logits: Tensor, k: int, score_fn: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Top-k / weights / aux partials from given fp32 logits [T, E]."""
    _on_gpu(logits)
    _require(logits.dtype == torch.float32 and logits.dim() == 2 and logits.is_contiguous(),
             "topk_from_logits: logits must be contiguous fp32 [T, E]")
    T, E = logits.shape
    dev = logits.device
    ids = torch.empty(T, k, device=dev, dtype=torch.int32)
    w = torch.empty(T, k, device=dev, dtype=torch.float32)
    pp = torch.empty(_nblk(T), E, device=dev, dtype=torch.float32)
    zp = torch.empty(_nblk(T), device=dev, dtype=torch.float32)
    st = nat.load().nt_moe_topk_from_logits(ptr(logits), T, E, k, score_fn, ptr(ids), ptr(w),
                                            ptr(pp), ptr(zp), _stream(dev))
    nat.check(st, "ntmoe::topk_from_logits")
    return ids, w, pp, zp


@topk_from_logits.register_fake
def _(logits, k, score_fn):
    T, E = logits.shape
    f = logits.new_empty
    return (f((T, k), dtype=torch.int32), f((T, k), dtype=torch.float32),
            f((_nblk(T), E), dtype=torch.float32), f((_nblk(T),), dtype=torch.float32))


# ---------------------------------------------------------------------------------------------
# route plan: histogram + scan + permute

@_custom_op("ntmoe::route_plan")
def route_plan(ids: Tensor, weights: Tensor, num_experts: int, x: Optional[Tensor],
               want_x_perm: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(counts [E], offsets [E+1], src_row [A], perm_w [A], combine_dest [T,k], combine_w [T,k],
    x_perm [A,d] or empty), A = T*k, in the order of mapping.T.nonzero()."""
    _on_gpu(ids, weights, x)
    _require(ids.dtype == torch.int32 and ids.dim() == 2 and ids.is_contiguous(),
             "route_plan: ids must be contiguous int32 [T, k]")
    _require(weights.dtype == torch.float32 and weights.shape == ids.shape and weights.is_contiguous(),
             "route_plan: weights must be contiguous fp32 [T, k]")
    T, k = ids.shape
    E = num_experts
    A = T * k
    dev = ids.device
    if want_x_perm:
        _require(x is not None and x.dtype == torch.bfloat16 and x.dim() == 2 and x.shape[0] == T
                 and x.stride(1) == 1, "route_plan: x must be bf16 [T, d] with contiguous rows")
    d = x.shape[1] if x is not None else 0
    counts = torch.empty(E, device=dev, dtype=torch.int32)
    offsets = torch.empty(E + 1, device=dev, dtype=torch.int32)
    src = torch.empty(A, device=dev, dtype=torch.int32)
    perm_w = torch.empty(A, device=dev, dtype=torch.float32)
    cdest = torch.empty(T, k, device=dev, dtype=torch.int32)
    cw = torch.empty(T, k, device=dev, dtype=torch.float32)
    x_perm = torch.empty((A, d) if want_x_perm else (0,), device=dev, dtype=torch.bfloat16)
    lib = nat.load()
    ws_bytes = lib.nt_moe_route_workspace_bytes(T, k, E)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    stream = _stream(dev)
    nat.check(lib.nt_moe_route_plan(ptr(x) if want_x_perm else None,
                                    x.stride(0) if want_x_perm else 0, ptr(ids), ptr(weights), T,
                                    d, k, E, ptr(counts), ptr(offsets), ptr(ws), ws_bytes,
                                    ptr(src), ptr(perm_w), ptr(cdest), ptr(cw),
                                    ptr(x_perm) if want_x_perm else None, stream),
              "ntmoe::route_plan")
    return counts, offsets, src, perm_w, cdest, cw, x_perm


@route_plan.register_fake
def _(ids, weights, num_experts, x, want_x_perm):
    T, k = ids.shape
    A = T * k
    d = x.shape[1] if x is not None else 0
    f = ids.new_empty
    return (f((num_experts,), dtype=torch.int32), f((num_experts + 1,), dtype=torch.int32),
            f((A,), dtype=torch.int32), f((A,), dtype=torch.float32), f((T, k), dtype=torch.int32),
            f((T, k), dtype=torch.float32),
            f((A, d) if want_x_perm else (0,), dtype=torch.bfloat16))


@_custom_op("ntmoe::router_plan")
def router_plan(x: Tensor, w_router_t: Tensor, bias: Optional[Tensor], k: int, score_fn: int,
                want_logits: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                            Tensor, Tensor, Tensor, Tensor]:
    """router followed by route_plan (without x_perm) in one C-ABI call and two launches: the
    same tensors, the same bits -- (logits, ids, weights, prob_partial, z_partial, counts,
    offsets, src_row, perm_w, combine_dest, combine_w)."""
    _on_gpu(x, w_router_t, bias)
    _require(x.dtype == torch.bfloat16 and x.dim() == 2, "router_plan: x must be bf16 [T, d]")
    _require(x.stride(1) == 1, "router_plan: x rows must be contiguous")
    _require(w_router_t.dtype == torch.float32 and w_router_t.is_contiguous(),
             "router_plan: w_router_t must be contiguous fp32 [d, E]")
    T, d = x.shape
    _require(w_router_t.shape[0] == d, "router_plan: w_router_t must be [d, E]")
    E = w_router_t.shape[1]
    if bias is not None:
        _require(bias.dtype == torch.float32 and bias.shape == (E,) and bias.is_contiguous(),
                 "router_plan: bias must be contiguous fp32 [E]")
    dev = x.device
    A = T * k
    f32, i32 = torch.float32, torch.int32
    logits = torch.empty((T, E) if want_logits else (0,), device=dev, dtype=f32)
    ids = torch.empty(T, k, device=dev, dtype=i32)
    w = torch.empty(T, k, device=dev, dtype=f32)
    pp = torch.empty(_nblk(T), E, device=dev, dtype=f32)
    zp = torch.empty(_nblk(T), device=dev, dtype=f32)
    counts = torch.empty(E, device=dev, dtype=i32)
    offsets = torch.empty(E + 1, device=dev, dtype=i32)
    src = torch.empty(A, device=dev, dtype=i32)
    perm_w = torch.empty(A, device=dev, dtype=f32)
    cdest = torch.empty(T, k, device=dev, dtype=i32)
    cw = torch.empty(T, k, device=dev, dtype=f32)
    lib = nat.load()
    ws_bytes = lib.nt_moe_router_plan_workspace_bytes(T, d, E, k)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    st = lib.nt_moe_router_plan(ptr(x), x.stride(0), ptr(w_router_t), ptr(bias), T, d, E, k,
                                score_fn, ptr(logits) if want_logits else None, ptr(ids), ptr(w),
                                ptr(pp), ptr(zp), ptr(counts), ptr(offsets), ptr(src),
                                ptr(perm_w), ptr(cdest), ptr(cw), ptr(ws), ws_bytes, _stream(dev))
    nat.check(st, "ntmoe::router_plan")
    return logits, ids, w, pp, zp, counts, offsets, src, perm_w, cdest, cw


@router_plan.register_fake
def _(x, w_router_t, bias, k, score_fn, want_logits):
    T, E = x.shape[0], w_router_t.shape[1]
    A = T * k
    f = x.new_empty
    f32, i32 = torch.float32, torch.int32
    return (f((T, E) if want_logits else (0,), dtype=f32), f((T, k), dtype=i32),
            f((T, k), dtype=f32), f((_nblk(T), E), dtype=f32), f((_nblk(T),), dtype=f32),
            f((E,), dtype=i32), f((E + 1,), dtype=i32), f((A,), dtype=i32), f((A,), dtype=f32),
            f((T, k), dtype=i32), f((T, k), dtype=f32))


# ---------------------------------------------------------------------------------------------
# grouped expert FFN

@_custom_op("ntmoe::grouped_ffn")
def grouped_ffn(a: Tensor, src_row: Optional[Tensor], seg_offsets: Tensor, w1: Tensor,
                w2: Tensor, activation: int, total_rows: int) -> tuple[Tensor, Tensor]:
    """(h [rows, H], y [rows, d]) for ragged segments; rows read a[src_row[r]] if given."""
    _on_gpu(a, src_row, seg_offsets, w1, w2)
    _require(a.dtype == torch.bfloat16 and a.dim() == 2 and a.stride(1) == 1,
             "grouped_ffn: a must be bf16 [*, d] with contiguous rows")
    _require(w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16 and w1.dim() == 3
             and w2.dim() == 3 and w1.is_contiguous() and w2.is_contiguous(),
             "grouped_ffn: w1 [S, F, d] and w2 [S, d, H] must be contiguous bf16")
    S, _, d = w1.shape
    H = w2.shape[2]
    F = 2 * H if activation == nat.ACT_SWIGLU else H
    _require(w1.shape == (S, F, d) and w2.shape == (S, d, H) and a.shape[1] == d,
             f"grouped_ffn: expected w1 [S,{F},{d}], w2 [S,{d},{H}], a [*, {d}]")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.shape == (S + 1,)
             and seg_offsets.is_contiguous(), "grouped_ffn: seg_offsets must be int32 [S+1]")
    if src_row is not None:
        _require(src_row.dtype == torch.int32 and src_row.is_contiguous(),
                 "grouped_ffn: src_row must be contiguous int32")
    dev = a.device
    h = torch.empty(total_rows, H, device=dev, dtype=torch.bfloat16)
    y = torch.empty(total_rows, d, device=dev, dtype=torch.bfloat16)
    lib = nat.load()
    ws_bytes = lib.nt_moe_grouped_gemm_workspace_bytes()
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    st = lib.nt_moe_grouped_ffn_bf16(ptr(a), a.stride(0), a.shape[0], ptr(src_row),
                                     ptr(seg_offsets), S, total_rows, ptr(w1), ptr(w2), d, H,
                                     activation, ptr(h), ptr(y), ptr(ws), ws_bytes, _stream(dev))
    nat.check(st, "ntmoe::grouped_ffn")
    return h, y


@grouped_ffn.register_fake
def _(a, src_row, seg_offsets, w1, w2, activation, total_rows):
    H, d = w2.shape[2], w1.shape[2]
    return (a.new_empty((total_rows, H)), a.new_empty((total_rows, d)))


@_custom_op("ntmoe::grouped_gemm")
def grouped_gemm(a: Tensor, src_row: Optional[Tensor], seg_offsets: Tensor, w: Tensor,
                 epilogue: int, total_rows: int) -> Tensor:
    """One grouped GEMM launch: c [rows, n_out] = epilogue(a_r . w_s^T) per ragged segment."""
    _on_gpu(a, src_row, seg_offsets, w)
    _require(a.dtype == torch.bfloat16 and a.dim() == 2 and a.stride(1) == 1,
             "grouped_gemm: a must be bf16 [*, K] with contiguous rows")
    _require(w.dtype == torch.bfloat16 and w.dim() == 3 and w.is_contiguous(),
             "grouped_gemm: w must be contiguous bf16 [S, rows, K]")
    S, rows, K = w.shape
    n_out = rows // 2 if epilogue == nat.EPI_SWIGLU else rows
    _require(a.shape[1] == K, "grouped_gemm: a and w disagree on K")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.shape == (S + 1,)
             and seg_offsets.is_contiguous(), "grouped_gemm: seg_offsets must be int32 [S+1]")
    if src_row is not None:
        _require(src_row.dtype == torch.int32 and src_row.is_contiguous(),
                 "grouped_gemm: src_row must be contiguous int32")
    c = torch.empty(total_rows, n_out, device=a.device, dtype=torch.bfloat16)
    lib = nat.load()
    ws_bytes = lib.nt_moe_grouped_gemm_workspace_bytes()
    ws = torch.empty(ws_bytes, device=a.device, dtype=torch.uint8)
    st = lib.nt_moe_grouped_gemm_bf16(ptr(a), a.stride(0), a.shape[0], ptr(src_row),
                                      ptr(seg_offsets), S, total_rows, ptr(w), K, n_out,
                                      epilogue, ptr(c), ptr(ws), ws_bytes, _stream(a.device))
    nat.check(st, "ntmoe::grouped_gemm")
    return c


@grouped_gemm.register_fake
def _(a, src_row, seg_offsets, w, epilogue, total_rows):
    rows = w.shape[1]
    return a.new_empty((total_rows, rows // 2 if epilogue == nat.EPI_SWIGLU else rows))


def plain_keep_supported(K, n_out):
    """Whether the plain-weight up projection can keep its fc1 pre-activations (the 256 x 256
    kernel: K >= 128, n_out a multiple of 8)."""
    return K >= 128 and n_out % 8 == 0


@_custom_op("ntmoe::grouped_gemm_keep")
def grouped_gemm_keep(a: Tensor, src_row: Optional[Tensor], seg_offsets: Tensor, w: Tensor,
                      epilogue: int, total_rows: int) -> tuple[Tensor, Tensor]:
    """(c, pre): grouped_gemm with the SwiGLU / ReLU^2 epilogue, plus the epilogue's input (the
    fc1 pre-activations, [rows, 2 n_out] or [rows, n_out]) for the backward."""
    _on_gpu(a, src_row, seg_offsets, w)
    _require(epilogue in (nat.EPI_SWIGLU, nat.EPI_RELU2),
             "grouped_gemm_keep: the epilogue must be SWIGLU or RELU2")
    _require(a.dtype == torch.bfloat16 and a.dim() == 2 and a.stride(1) == 1,
             "grouped_gemm_keep: a must be bf16 [*, K] with contiguous rows")
    _require(w.dtype == torch.bfloat16 and w.dim() == 3 and w.is_contiguous(),
             "grouped_gemm_keep: w must be contiguous bf16 [S, rows, K]")
    S, rows, K = w.shape
    n_out = rows // 2 if epilogue == nat.EPI_SWIGLU else rows
    _require(a.shape[1] == K, "grouped_gemm_keep: a and w disagree on K")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.shape == (S + 1,)
             and seg_offsets.is_contiguous(), "grouped_gemm_keep: seg_offsets must be int32 [S+1]")
    if src_row is not None:
        _require(src_row.dtype == torch.int32 and src_row.is_contiguous(),
                 "grouped_gemm_keep: src_row must be contiguous int32")
    c = torch.empty(total_rows, n_out, device=a.device, dtype=torch.bfloat16)
    pre = torch.empty(total_rows, rows, device=a.device, dtype=torch.bfloat16)
    st = nat.load().nt_moe_grouped_gemm_bf16_keep(
        ptr(a), a.stride(0), a.shape[0], ptr(src_row), ptr(seg_offsets), S, total_rows, ptr(w), K,
        n_out, epilogue, ptr(c), ptr(pre), _stream(a.device))
    nat.check(st, "ntmoe::grouped_gemm_keep")
    return c, pre


@grouped_gemm_keep.register_fake
def _(a, src_row, seg_offsets, w, epilogue, total_rows):
    S, rows, K = w.shape
    n_out = rows // 2 if epilogue == nat.EPI_SWIGLU else rows
    return (a.new_empty(total_rows, n_out), a.new_empty(total_rows, rows))


@_custom_op("ntmoe::pack_expert_weights")
def pack_expert_weights(w: Tensor, epilogue: int) -> Tensor:
    """Expert weights [S, rows, K] bf16 rearranged for grouped_gemm_packed (same size)."""
    _on_gpu(w)
    _require(w.dtype == torch.bfloat16 and w.dim() == 3 and w.is_contiguous(),
             "pack_expert_weights: w must be contiguous bf16 [S, rows, K]")
    S, R, K = w.shape
    out = torch.empty_like(w)
    st = nat.load().nt_moe_pack_expert_weights_bf16(ptr(w), S, R, K, epilogue, ptr(out),
                                                    _stream(w.device))
    nat.check(st, "ntmoe::pack_expert_weights")
    return out


@pack_expert_weights.register_fake
def _(w, epilogue):
    return torch.empty_like(w)


@_custom_op("ntmoe::convert_expert_weights")
def convert_expert_weights(w: Tensor, want_out: bool, want_t: bool) -> tuple[Tensor, Tensor]:
    """fp32 [S, R, K] -> (bf16 [S, R, K] or empty, bf16 [S, K, R] or empty), one read of w."""
    _on_gpu(w)
    _require(w.dtype == torch.float32 and w.dim() == 3 and w.is_contiguous(),
             "convert_expert_weights: w must be contiguous fp32 [S, R, K]")
    S, R, K = w.shape
    out = torch.empty((S, R, K) if want_out else (0,), device=w.device, dtype=torch.bfloat16)
    out_t = torch.empty((S, K, R) if want_t else (0,), device=w.device, dtype=torch.bfloat16)
    st = nat.load().nt_moe_convert_expert_weights(ptr(w), S, R, K,
                                                  ptr(out) if want_out else None,
                                                  ptr(out_t) if want_t else None,
                                                  _stream(w.device))
    nat.check(st, "ntmoe::convert_expert_weights")
    return out, out_t


@convert_expert_weights.register_fake
def _(w, want_out, want_t):
    S, R, K = w.shape
    return (w.new_empty((S, R, K) if want_out else (0,), dtype=torch.bfloat16),
            w.new_empty((S, K, R) if want_t else (0,), dtype=torch.bfloat16))


def first_layout(E, Fs):
    """(Ep, Kc) of the backward's concatenated first operand [S^T | hi | lo | hi] for E experts
    and a shared expert of Fs fc1 rows (0 without one): E padded to 32, the width to 64."""
    Ep = _round_up(E, 32)
    return Ep, _round_up(Fs + 3 * Ep, 64)


@_custom_op("ntmoe::router_operands")
def router_operands(w: Tensor, dp: int, shared_w1: Optional[Tensor], want_first: bool
                    ) -> tuple[Tensor, Tensor]:
    """From the fp32 router weight w [E, d]: (w_router_t fp32 [dp, E], rows past d zero; and,
    with want_first, the backward's first operand bf16 [1, dp, Kc] = [S^T | hi | lo | hi | 0]
    for the shared expert's W1 S bf16 [Fs, dp] (or none), hi / lo the two-term bf16 split of
    w_router_t, (Ep, Kc) = first_layout(E, Fs); else an empty tensor), in one kernel."""
    _on_gpu(w, shared_w1)
    _require(w.dtype == torch.float32 and w.dim() == 2 and w.stride(1) == 1,
             "router_operands: w must be fp32 [E, d] with contiguous rows")
    E, d = w.shape
    _require(dp >= d, "router_operands: dp must be >= d")
    Fs = 0
    if want_first and shared_w1 is not None:
        _require(shared_w1.dtype == torch.bfloat16 and shared_w1.dim() == 2
                 and shared_w1.shape[1] == dp and shared_w1.stride(1) == 1,
                 "router_operands: shared_w1 must be bf16 [Fs, dp] with contiguous rows")
        Fs = shared_w1.shape[0]
    Ep, Kc = first_layout(E, Fs)
    rt = torch.empty(dp, E, device=w.device, dtype=torch.float32)
    first = torch.empty((1, dp, Kc) if want_first else (0,), device=w.device,
                        dtype=torch.bfloat16)
    st = nat.load().nt_moe_router_operands(
        ptr(w), w.stride(0), E, d, dp, ptr(shared_w1) if Fs else None,
        shared_w1.stride(0) if Fs else 0, Fs, ptr(rt), ptr(first) if want_first else None,
        Ep, Kc, _stream(w.device))
    nat.check(st, "ntmoe::router_operands")
    return rt, first


@router_operands.register_fake
def _(w, dp, shared_w1, want_first):
    E = w.shape[0]
    Fs = shared_w1.shape[0] if (want_first and shared_w1 is not None) else 0
    Kc = first_layout(E, Fs)[1]
    return (w.new_empty(dp, E), w.new_empty((1, dp, Kc) if want_first else (0,),
                                            dtype=torch.bfloat16))


@_custom_op("ntmoe::convert_pack_expert_weights")
def convert_pack_expert_weights(w: Tensor, epilogue: int, want_out: bool, want_t: bool,
                                want_packed: bool, want_packed_t: bool
                                ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """fp32 [S, R, K] -> (bf16 w, bf16 w^T [S, K, R], w packed for `epilogue`, w^T packed as a
    plain projection), each or an empty tensor, from one read of w; the packed ones equal
    pack_expert_weights of the bf16 copies bit for bit."""
    _on_gpu(w)
    _require(w.dtype == torch.float32 and w.dim() == 3 and w.is_contiguous(),
             "convert_pack_expert_weights: w must be contiguous fp32 [S, R, K]")
    S, R, K = w.shape
    mk = lambda want, shape: torch.empty(shape if want else (0,), device=w.device,
                                         dtype=torch.bfloat16)
    out, out_t = mk(want_out, (S, R, K)), mk(want_t, (S, K, R))
    pk, pk_t = mk(want_packed, (S, R, K)), mk(want_packed_t, (S, K, R))
    st = nat.load().nt_moe_convert_expert_weights_packed(
        ptr(w), S, R, K, ptr(out) if want_out else None, ptr(out_t) if want_t else None,
        ptr(pk) if want_packed else None, int(epilogue), ptr(pk_t) if want_packed_t else None,
        _stream(w.device))
    nat.check(st, "ntmoe::convert_pack_expert_weights")
    return out, out_t, pk, pk_t


@convert_pack_expert_weights.register_fake
def _(w, epilogue, want_out, want_t, want_packed, want_packed_t):
    S, R, K = w.shape
    mk = lambda want, shape: w.new_empty(shape if want else (0,), dtype=torch.bfloat16)
    return (mk(want_out, (S, R, K)), mk(want_t, (S, K, R)), mk(want_packed, (S, R, K)),
            mk(want_packed_t, (S, K, R)))


def packable(K, n_out, epilogue):
    """Whether a [*, n_out or 2 n_out, K] weight stack qualifies for the packed GEMM."""
    return K >= 256 and K % 64 == 0 and n_out % (16 if epilogue == nat.EPI_SWIGLU else 32) == 0


def prefers_packed(K, n_out, epilogue, repacked_each_step=True):
    """Whether the layer packs a projection. Weights packed once (inference): whenever packable.
    Weights repacked after every update (training): only with an even count of 64-wide K steps.
    An odd count (K = 320, the T3 cell's down projection and fc1 dgrad) runs a sixth step per
    tile that multiplies nothing; there the packed kernel measured 176 us against the 256 x 256
    plain-weight kernel's 210 us, less than the ~80 us repack of the [256, 1280, 320] weights
    that each training step would add."""
    return packable(K, n_out, epilogue) and (K % 128 == 0 or not repacked_each_step)


@_custom_op("ntmoe::grouped_gemm_packed")
def grouped_gemm_packed(a: Tensor, src_row: Optional[Tensor], seg_offsets: Tensor,
                        w_packed: Tensor, epilogue: int, total_rows: int) -> Tensor:
    """grouped_gemm on weights packed by pack_expert_weights with the same epilogue."""
    _on_gpu(a, src_row, seg_offsets, w_packed)
    _require(a.dtype == torch.bfloat16 and a.dim() == 2 and a.stride(1) == 1,
             "grouped_gemm_packed: a must be bf16 [*, K] with contiguous rows")
    _require(w_packed.dtype == torch.bfloat16 and w_packed.dim() == 3 and w_packed.is_contiguous(),
             "grouped_gemm_packed: w_packed must be contiguous bf16 [S, rows, K]")
    S, rows, K = w_packed.shape
    n_out = rows // 2 if epilogue == nat.EPI_SWIGLU else rows
    _require(a.shape[1] == K, "grouped_gemm_packed: a and w disagree on K")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.shape == (S + 1,)
             and seg_offsets.is_contiguous(), "grouped_gemm_packed: seg_offsets must be int32 [S+1]")
    if src_row is not None:
        _require(src_row.dtype == torch.int32 and src_row.is_contiguous(),
                 "grouped_gemm_packed: src_row must be contiguous int32")
    c = torch.empty(total_rows, n_out, device=a.device, dtype=torch.bfloat16)
    st = nat.load().nt_moe_grouped_gemm_bf16_packed(
        ptr(a), a.stride(0), a.shape[0], ptr(src_row), ptr(seg_offsets), S, total_rows,
        ptr(w_packed), K, n_out, epilogue, ptr(c), _stream(a.device))
    nat.check(st, "ntmoe::grouped_gemm_packed")
    return c


@grouped_gemm_packed.register_fake
def _(a, src_row, seg_offsets, w_packed, epilogue, total_rows):
    rows = w_packed.shape[1]
    return a.new_empty((total_rows, rows // 2 if epilogue == nat.EPI_SWIGLU else rows))


@_custom_op("ntmoe::grouped_gemm_packed_keep")
def grouped_gemm_packed_keep(a: Tensor, src_row: Optional[Tensor], seg_offsets: Tensor,
                             w_packed: Tensor, epilogue: int,
                             total_rows: int) -> tuple[Tensor, Tensor]:
    """(c, pre): grouped_gemm_packed with the SwiGLU / ReLU^2 epilogue, plus the epilogue's input
    (the fc1 pre-activations, [rows, 2 n_out] or [rows, n_out]) for the backward."""
    _on_gpu(a, src_row, seg_offsets, w_packed)
    _require(epilogue in (nat.EPI_SWIGLU, nat.EPI_RELU2),
             "grouped_gemm_packed_keep: the epilogue must be SWIGLU or RELU2")
    _require(a.dtype == torch.bfloat16 and a.dim() == 2 and a.stride(1) == 1,
             "grouped_gemm_packed_keep: a must be bf16 [*, K] with contiguous rows")
    _require(w_packed.dtype == torch.bfloat16 and w_packed.dim() == 3 and w_packed.is_contiguous(),
             "grouped_gemm_packed_keep: w_packed must be contiguous bf16 [S, rows, K]")
    S, rows, K = w_packed.shape
    n_out = rows // 2 if epilogue == nat.EPI_SWIGLU else rows
    _require(a.shape[1] == K, "grouped_gemm_packed_keep: a and w disagree on K")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.shape == (S + 1,)
             and seg_offsets.is_contiguous(),
             "grouped_gemm_packed_keep: seg_offsets must be int32 [S+1]")
    if src_row is not None:
        _require(src_row.dtype == torch.int32 and src_row.is_contiguous(),
                 "grouped_gemm_packed_keep: src_row must be contiguous int32")
    c = torch.empty(total_rows, n_out, device=a.device, dtype=torch.bfloat16)
    pre = torch.empty(total_rows, rows, device=a.device, dtype=torch.bfloat16)
    st = nat.load().nt_moe_grouped_gemm_bf16_packed_keep(
        ptr(a), a.stride(0), a.shape[0], ptr(src_row), ptr(seg_offsets), S, total_rows,
        ptr(w_packed), K, n_out, epilogue, ptr(c), ptr(pre), _stream(a.device))
    nat.check(st, "ntmoe::grouped_gemm_packed_keep")
    return c, pre


@grouped_gemm_packed_keep.register_fake
def _(a, src_row, seg_offsets, w_packed, epilogue, total_rows):
    S, rows, K = w_packed.shape
    n_out = rows // 2 if epilogue == nat.EPI_SWIGLU else rows
    return (a.new_empty(total_rows, n_out), a.new_empty(total_rows, rows))


# ---------------------------------------------------------------------------------------------
# fp8 (OCP e4m3fn bytes held in uint8 tensors)

@_custom_op("ntmoe::quantize_fp8_rowwise")
def quantize_fp8_rowwise(x: Tensor) -> tuple[Tensor, Tensor]:
    """(q uint8 [rows, d] e4m3 codes, scale fp32 [rows]) with s = amax / 448 per row."""
    _on_gpu(x)
    _require(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1,
             "quantize_fp8_rowwise: x must be bf16 [rows, d] with contiguous rows")
    rows, d = x.shape
    # rows of q stay 32-byte aligned for the fp8 GEMM's 32-byte operand loads
    _require(d % 32 == 0, "quantize_fp8_rowwise: d must be a multiple of 32")
    q = torch.empty(rows, d, device=x.device, dtype=torch.uint8)
    scale = torch.empty(rows, device=x.device, dtype=torch.float32)
    st = nat.load().nt_moe_quantize_fp8_rowwise(ptr(x), x.stride(0), rows, d, ptr(q), d,
                                                ptr(scale), _stream(x.device))
    nat.check(st, "ntmoe::quantize_fp8_rowwise")
    return q, scale


@quantize_fp8_rowwise.register_fake
def _(x):
    rows, d = x.shape
    return (x.new_empty((rows, d), dtype=torch.uint8), x.new_empty((rows,), dtype=torch.float32))


@_custom_op("ntmoe::quantize_fp8_blockwise")
def quantize_fp8_blockwise(w: Tensor) -> tuple[Tensor, Tensor]:
    """(q uint8 [S, R, C] e4m3 codes, scale fp32 [S, R/128, C/128]) of fp32 w [S, R, C]."""
    _on_gpu(w)
    _require(w.dtype == torch.float32 and w.dim() == 3 and w.is_contiguous(),
             "quantize_fp8_blockwise: w must be contiguous fp32 [S, R, C]")
    S, R, C = w.shape
    q = torch.empty(S, R, C, device=w.device, dtype=torch.uint8)
    scale = torch.empty(S, R // 128, C // 128, device=w.device, dtype=torch.float32)
    st = nat.load().nt_moe_quantize_fp8_blockwise(ptr(w), S, R, C, ptr(q), ptr(scale),
                                                  _stream(w.device))
    nat.check(st, "ntmoe::quantize_fp8_blockwise")
    return q, scale


@quantize_fp8_blockwise.register_fake
def _(w):
    S, R, C = w.shape
    return (w.new_empty((S, R, C), dtype=torch.uint8),
            w.new_empty((S, R // 128, C // 128), dtype=torch.float32))


@_custom_op("ntmoe::pack_expert_weights_fp8")
def pack_expert_weights_fp8(w: Tensor, epilogue: int) -> Tensor:
    """e4m3 expert weights [S, rows, K] (uint8) rearranged for grouped_gemm_fp8(packed=True)."""
    _on_gpu(w)
    _require(w.dtype == torch.uint8 and w.dim() == 3 and w.is_contiguous(),
             "pack_expert_weights_fp8: w must be contiguous uint8 (e4m3) [S, rows, K]")
    S, R, K = w.shape
    out = torch.empty_like(w)
    st = nat.load().nt_moe_pack_expert_weights_fp8(ptr(w), S, R, K, epilogue, ptr(out),
                                                   _stream(w.device))
    nat.check(st, "ntmoe::pack_expert_weights_fp8")
    return out


@pack_expert_weights_fp8.register_fake
def _(w, epilogue):
    return torch.empty_like(w)


@_custom_op("ntmoe::grouped_gemm_fp8")
def grouped_gemm_fp8(a: Tensor, a_scale: Tensor, src_row: Optional[Tensor], seg_offsets: Tensor,
                     w: Tensor, w_scale: Tensor, epilogue: int, total_rows: int,
                     packed: bool = False) -> Tensor:
    """c bf16 [rows, n_out] = epilogue(a_scale . sum_kb w_scale . (a_q . w_q^T)_kb) per segment;
    with `packed`, w comes from pack_expert_weights_fp8 (same epilogue)."""
    _on_gpu(a, a_scale, src_row, seg_offsets, w, w_scale)
    _require(a.dtype == torch.uint8 and a.dim() == 2 and a.stride(1) == 1,
             "grouped_gemm_fp8: a must be uint8 (e4m3) [*, K] with contiguous rows")
    _require(w.dtype == torch.uint8 and w.dim() == 3 and w.is_contiguous(),
             "grouped_gemm_fp8: w must be contiguous uint8 (e4m3) [S, R, K]")
    S, R, K = w.shape
    n_out = R // 2 if epilogue == nat.EPI_SWIGLU else R
    _require(a.shape[1] == K, "grouped_gemm_fp8: a and w disagree on K")
    _require(a_scale.dtype == torch.float32 and a_scale.shape == (a.shape[0],)
             and a_scale.is_contiguous(), "grouped_gemm_fp8: a_scale must be fp32 [a_rows]")
    _require(w_scale.dtype == torch.float32 and w_scale.shape == (S, R // 128, K // 128)
             and w_scale.is_contiguous(), "grouped_gemm_fp8: w_scale must be fp32 [S, R/128, K/128]")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.shape == (S + 1,)
             and seg_offsets.is_contiguous(), "grouped_gemm_fp8: seg_offsets must be int32 [S+1]")
    if src_row is not None:
        _require(src_row.dtype == torch.int32 and src_row.is_contiguous(),
                 "grouped_gemm_fp8: src_row must be contiguous int32")
    c = torch.empty(total_rows, n_out, device=a.device, dtype=torch.bfloat16)
    fn = (nat.load().nt_moe_grouped_gemm_fp8_packed if packed
          else nat.load().nt_moe_grouped_gemm_fp8)
    st = fn(ptr(a), a.stride(0), a.shape[0], ptr(a_scale), ptr(src_row), ptr(seg_offsets), S,
            total_rows, ptr(w), ptr(w_scale), K, n_out, epilogue, ptr(c), _stream(a.device))
    nat.check(st, "ntmoe::grouped_gemm_fp8")
    return c


@grouped_gemm_fp8.register_fake
def _(a, a_scale, src_row, seg_offsets, w, w_scale, epilogue, total_rows, packed=False):
    R = w.shape[1]
    return a.new_empty((total_rows, R // 2 if epilogue == nat.EPI_SWIGLU else R),
                       dtype=torch.bfloat16)


# ---------------------------------------------------------------------------------------------
# combine + aux

@_custom_op("ntmoe::combine_aux")
def combine_aux(y: Tensor, combine_dest: Tensor, combine_w: Tensor, shared_y: Optional[Tensor],
                prob_partial: Tensor, z_partial: Tensor, counts: Tensor, aux_coeff: float,
                z_coeff: float) -> tuple[Tensor, Tensor]:
    """(out [T, d] bf16, aux fp32 [3] = {lb + z, lb, z})."""
    _on_gpu(y, combine_dest, combine_w, shared_y, prob_partial, z_partial, counts)
    _require(y.dtype == torch.bfloat16 and y.dim() == 2 and y.is_contiguous(),
             "combine_aux: y must be contiguous bf16 [A, d]")
    T, k = combine_dest.shape
    d = y.shape[1]
    E = counts.shape[0]
    _require(combine_dest.dtype == torch.int32 and combine_dest.is_contiguous()
             and combine_w.dtype == torch.float32 and combine_w.shape == (T, k)
             and combine_w.is_contiguous(), "combine_aux: bad combine_dest / combine_w")
    _require(counts.dtype == torch.int32 and prob_partial.shape == (_nblk(T), E)
             and z_partial.shape == (_nblk(T),), "combine_aux: bad aux partials")
    if shared_y is not None:
        _require(shared_y.dtype == torch.bfloat16 and shared_y.shape == (T, d)
                 and shared_y.stride(1) == 1, "combine_aux: shared_y must be bf16 [T, d]")
    dev = y.device
    out = torch.empty(T, d, device=dev, dtype=torch.bfloat16)
    aux = torch.empty(3, device=dev, dtype=torch.float32)
    st = nat.load().nt_moe_combine_aux(
        ptr(y), ptr(combine_dest), ptr(combine_w), T, d, k, ptr(shared_y),
        shared_y.stride(0) if shared_y is not None else 0, ptr(out), out.stride(0),
        ptr(prob_partial), ptr(z_partial), ptr(counts), E, float(aux_coeff), float(z_coeff),
        ptr(aux), _stream(dev))
    nat.check(st, "ntmoe::combine_aux")
    return out, aux


@combine_aux.register_fake
def _(y, combine_dest, combine_w, shared_y, prob_partial, z_partial, counts, aux_coeff, z_coeff):
    T = combine_dest.shape[0]
    return y.new_empty((T, y.shape[1])), y.new_empty((3,), dtype=torch.float32)


# ---------------------------------------------------------------------------------------------
# the whole layer

_SEGMENTS = {}


def _whole_batch_segment(T, device):
    """Device tensor [0, T]: the shared expert's single segment (cached: no per-call upload)."""
    key = (T, device)
    seg = _SEGMENTS.get(key)
    if seg is None:
        seg = torch.tensor([0, T], device=device, dtype=torch.int32)
        if len(_SEGMENTS) < 64:
            _SEGMENTS[key] = seg
    return seg


def moe_forward(x, w_router_t, w1, w2, *, top_k, score_fn=nat.SCORE_SOFTMAX,
                activation=nat.ACT_SWIGLU, aux_coeff=0.01, z_coeff=0.001, logit_bias=None,
                shared_w1=None, shared_w2=None, want_logits=False, permute_rows=False,
                w1_scale=None, w2_scale=None, shared_w1_scale=None, shared_w2_scale=None,
                packed=False, mark=None, keep=False):
    """The MoE layer forward on the GPU: router -> route plan -> grouped GEMMs -> combine + aux.

    x bf16 [T, d]; w_router_t fp32 [d, E]; w1 bf16 [E, F, d] (F = 2H for SwiGLU, H for ReLU^2);
    w2 bf16 [E, d, H]; optional shared expert shared_w1 [1, Fs, d], shared_w2 [1, d, Hs].
    Returns (out [T, d] bf16, aux fp32 [3] = {lb + z, lb, z}, state with the routing tensors).
    With permute_rows the token rows are first moved into expert order by the permute kernel
    (x_perm); by default the up-projection GEMM gathers them itself.
    packed: w1 (and shared_w1) were packed by pack_expert_weights (bf16) or
    pack_expert_weights_fp8 (e4m3) with the up epilogue, w2 (and shared_w2) with EPI_NONE; the
    packed grouped GEMMs run both projections. For bf16 also a pair (up, down): which of the
    two projections' weights are packed (the other ones plain [E, rows, K]).
    fp8 experts: pass w1/w2 (and the shared expert's) as uint8 e4m3 codes with their 128 x 128
    block scales (w*_scale, from quantize_fp8_blockwise); the token rows and the intermediate
    h are then quantised per row and both projections run on the fp8 grouped GEMM.
    `mark(name)`, when given, is called after each stage is enqueued (used to place timing
    events on the stream; without permute_rows the router and the route plan are one call, so
    the "router" stage holds both and "route_plan" is empty). keep (bf16 experts): the state also holds what moe_backward reads
    (h, y, the shared expert's h, the router's aux partials and the fc1 pre-activations of
    the routed and the shared expert from their up projections' launches, with packed weights
    or plain ones that plain_keep_supported takes; otherwise moe_backward recomputes them).
    """
    T = x.shape[0]
    E = w_router_t.shape[1]
    A = T * top_k
    mark = mark or (lambda name: None)
    if T == 0:
        dev = x.device
        i32, f32 = torch.int32, torch.float32
        empty = lambda *shape, dtype=i32: torch.empty(shape, device=dev, dtype=dtype)
        state = dict(logits=empty(0, E, dtype=f32), ids=empty(0, top_k),
                     weights=empty(0, top_k, dtype=f32), counts=torch.zeros(E, device=dev, dtype=i32),
                     offsets=torch.zeros(E + 1, device=dev, dtype=i32), src_row=empty(0),
                     perm_w=empty(0, dtype=f32), combine_dest=empty(0, top_k),
                     combine_w=empty(0, top_k, dtype=f32))
        return x.new_empty(0, x.shape[1]), torch.zeros(3, device=dev, dtype=f32), state
    if permute_rows:
        logits, ids, w, pp, zp = router.raw(x, w_router_t, logit_bias, top_k, score_fn,
                                            want_logits)
        mark("router")
        counts, offsets, src, perm_w, cdest, cw, x_perm = route_plan.raw(ids, w, E, x, True)
    else:  # one call, two launches: the router's top-k counts for the plan
        (logits, ids, w, pp, zp, counts, offsets, src, perm_w, cdest,
         cw) = router_plan.raw(x, w_router_t, logit_bias, top_k, score_fn, want_logits)
        x_perm = None
        mark("router")
    mark("route_plan")
    up_epi = nat.EPI_SWIGLU if activation == nat.ACT_SWIGLU else nat.EPI_RELU2
    if w1.dtype == torch.uint8:
        _require(w1_scale is not None and w2_scale is not None,
                 "moe_forward: fp8 weights need w1_scale and w2_scale")
        _require(isinstance(packed, bool), "moe_forward: fp8 weights take packed=True or False")
        xq, xs = quantize_fp8_rowwise.raw(x)
        mark("quantize")
        h = grouped_gemm_fp8.raw(xq, xs, src, offsets, w1, w1_scale, up_epi, A, packed)
        mark("gemm_up")
        hq, hs = quantize_fp8_rowwise.raw(h)
        y = grouped_gemm_fp8.raw(hq, hs, None, offsets, w2, w2_scale, nat.EPI_NONE, A, packed)
        mark("gemm_down")
        shared_y = None
        if shared_w1 is not None:
            seg = _whole_batch_segment(T, x.device)
            hs_ = grouped_gemm_fp8.raw(xq, xs, None, seg, shared_w1, shared_w1_scale, up_epi, T,
                                   packed)
            hsq, hss = quantize_fp8_rowwise.raw(hs_)
            shared_y = grouped_gemm_fp8.raw(hsq, hss, None, seg, shared_w2, shared_w2_scale,
                                        nat.EPI_NONE, T, packed)
            mark("shared")
        out, aux = combine_aux.raw(y, cdest, cw, shared_y, pp, zp, counts, aux_coeff, z_coeff)
        mark("combine")
        state = dict(logits=logits, ids=ids, weights=w, counts=counts, offsets=offsets,
                     src_row=src, perm_w=perm_w, combine_dest=cdest, combine_w=cw, x_q=xq,
                     x_scale=xs)
        return out, aux, state
    packed_up, packed_down = (packed, packed) if isinstance(packed, bool) else packed
    gemm_up = grouped_gemm_packed.raw if packed_up else grouped_gemm.raw
    gemm_down = grouped_gemm_packed.raw if packed_down else grouped_gemm.raw

    def up(a, rows_src, offs, w, rows):
        """The up projection; with keep, also the backward's fc1 pre-activations from the same
        launch where the kernel can store them (else None: the backward recomputes them)."""
        if keep and packed_up:
            return grouped_gemm_packed_keep.raw(a, rows_src, offs, w, up_epi, rows)
        if keep and plain_keep_supported(
                w.shape[2], w.shape[1] // 2 if up_epi == nat.EPI_SWIGLU else w.shape[1]):
            return grouped_gemm_keep.raw(a, rows_src, offs, w, up_epi, rows)
        return gemm_up(a, rows_src, offs, w, up_epi, rows), None

    if permute_rows:
        h, fc1 = gemm_up(x_perm, None, offsets, w1, up_epi, A), None
    else:
        h, fc1 = up(x, src, offsets, w1, A)
    mark("gemm_up")
    y = gemm_down(h, None, offsets, w2, nat.EPI_NONE, A)
    mark("gemm_down")
    shared_y = hs = fc1s = None
    if shared_w1 is not None:
        seg = _whole_batch_segment(T, x.device)
        hs, fc1s = up(x, None, seg, shared_w1, T)
        shared_y = gemm_down(hs, None, seg, shared_w2, nat.EPI_NONE, T)
        mark("shared")
    out, aux = combine_aux.raw(y, cdest, cw, shared_y, pp, zp, counts, aux_coeff, z_coeff)
    mark("combine")
    state = dict(logits=logits, ids=ids, weights=w, counts=counts, offsets=offsets, src_row=src,
                 perm_w=perm_w, combine_dest=cdest, combine_w=cw)
    if keep:
        state.update(h=h, y=y, shared_h=hs, prob_partial=pp, z_partial=zp, fc1=fc1,
                     shared_fc1=fc1s)
    return out, aux, state


# ---------------------------------------------------------------------------------------------
# backward (bf16 experts)

@_custom_op("ntmoe::combine_bwd")
def combine_bwd(grad_out: Tensor, y: Tensor, ids: Tensor, combine_dest: Tensor,
                combine_w: Tensor) -> tuple[Tensor, Tensor]:
    """(grad_y bf16 [T*k, d] expert-major, grad_w fp32 [T, k] in top-k slot order)."""
    _on_gpu(grad_out, y, ids, combine_dest, combine_w)
    T, k = ids.shape
    _require(grad_out.dtype == torch.bfloat16 and grad_out.dim() == 2 and grad_out.shape[0] == T
             and grad_out.stride(1) == 1, "combine_bwd: grad_out must be bf16 [T, d]")
    d = grad_out.shape[1]
    _require(y.dtype == torch.bfloat16 and y.shape == (T * k, d) and y.is_contiguous(),
             "combine_bwd: y must be contiguous bf16 [T*k, d]")
    _require(ids.dtype == torch.int32 and ids.is_contiguous() and combine_dest.dtype == torch.int32
             and combine_dest.shape == (T, k) and combine_dest.is_contiguous()
             and combine_w.dtype == torch.float32 and combine_w.shape == (T, k)
             and combine_w.is_contiguous(), "combine_bwd: bad ids / combine_dest / combine_w")
    dev = y.device
    gy = torch.empty(T * k, d, device=dev, dtype=torch.bfloat16)
    gw = torch.empty(T, k, device=dev, dtype=torch.float32)
    st = nat.load().nt_moe_combine_bwd(ptr(grad_out), grad_out.stride(0), ptr(y), ptr(ids),
                                       ptr(combine_dest), ptr(combine_w), T, d, k, ptr(gy),
                                       ptr(gw), _stream(dev))
    nat.check(st, "ntmoe::combine_bwd")
    return gy, gw


@combine_bwd.register_fake
def _(grad_out, y, ids, combine_dest, combine_w):
    T, k = ids.shape
    return (y.new_empty(T * k, grad_out.shape[1]),
            y.new_empty((T, k), dtype=torch.float32))


@_custom_op("ntmoe::act_bwd")
def act_bwd(fc1: Tensor, grad_h: Tensor, activation: int) -> Tensor:
    """grad of the fc1 pre-activations [rows, F] from grad_h [rows, H]."""
    _on_gpu(fc1, grad_h)
    _require(fc1.dtype == torch.bfloat16 and grad_h.dtype == torch.bfloat16 and fc1.is_contiguous()
             and grad_h.is_contiguous() and fc1.dim() == 2 and grad_h.dim() == 2,
             "act_bwd: fc1 and grad_h must be contiguous bf16 matrices")
    rows, H = grad_h.shape
    F = 2 * H if activation == nat.ACT_SWIGLU else H
    _require(fc1.shape == (rows, F), "act_bwd: fc1 must be [rows, 2H] (SwiGLU) or [rows, H]")
    out = torch.empty_like(fc1)
    st = nat.load().nt_moe_act_bwd(ptr(fc1), ptr(grad_h), rows, H, activation, ptr(out),
                                   _stream(fc1.device))
    nat.check(st, "ntmoe::act_bwd")
    return out


@act_bwd.register_fake
def _(fc1, grad_h, activation):
    return torch.empty_like(fc1)


@_custom_op("ntmoe::backward_first_operand")
def backward_first_operand(grad_logits: Tensor, dfc1s: Optional[Tensor], Ep: int,
                           Kc: int) -> Tensor:
    """bf16 [T, Kc] rows [dfc1s | g_hi | g_hi | g_lo | 0], g = grad_logits split as
    split_bf16 does, each g block Ep wide (columns past E zero); dfc1s bf16 [T, Fs] or None."""
    _on_gpu(grad_logits, dfc1s)
    _require(grad_logits.dtype == torch.float32 and grad_logits.dim() == 2
             and grad_logits.is_contiguous(), "backward_first_operand: grad_logits must be "
             "contiguous fp32 [T, E]")
    T, E = grad_logits.shape
    Fs = 0
    if dfc1s is not None:
        _require(dfc1s.dtype == torch.bfloat16 and dfc1s.dim() == 2 and dfc1s.shape[0] == T
                 and dfc1s.is_contiguous(), "backward_first_operand: dfc1s must be contiguous "
                 "bf16 [T, Fs]")
        Fs = dfc1s.shape[1]
    out = torch.empty(T, Kc, device=grad_logits.device, dtype=torch.bfloat16)
    st = nat.load().nt_moe_backward_first_operand(ptr(grad_logits), E, ptr(dfc1s), Fs, T, Ep, Kc,
                                                  ptr(out), _stream(grad_logits.device))
    nat.check(st, "ntmoe::backward_first_operand")
    return out


@backward_first_operand.register_fake
def _(grad_logits, dfc1s, Ep, Kc):
    return grad_logits.new_empty(grad_logits.shape[0], Kc, dtype=torch.bfloat16)


@_custom_op("ntmoe::router_bwd")
def router_bwd(logits: Tensor, ids: Tensor, weights: Tensor, grad_w: Tensor, counts: Tensor,
               score_fn: int, grad_aux: Optional[Tensor], aux_coeff: float,
               z_coeff: float) -> Tensor:
    """grad_logits fp32 [T, E] (routing-weight and aux/z-loss terms)."""
    _on_gpu(logits, ids, weights, grad_w, counts, grad_aux)
    T, E = logits.shape
    k = ids.shape[1]
    _require(logits.dtype == torch.float32 and logits.is_contiguous(),
             "router_bwd: logits must be contiguous fp32 [T, E]")
    _require(ids.dtype == torch.int32 and ids.shape == (T, k) and ids.is_contiguous()
             and weights.dtype == torch.float32 and weights.shape == (T, k)
             and weights.is_contiguous() and grad_w.dtype == torch.float32
             and grad_w.shape == (T, k) and grad_w.is_contiguous(),
             "router_bwd: bad ids / weights / grad_w")
    _require(counts.dtype == torch.int32 and counts.shape == (E,), "router_bwd: bad counts")
    if grad_aux is not None:
        _require(grad_aux.dtype == torch.float32 and grad_aux.shape == (3,)
                 and grad_aux.is_contiguous(), "router_bwd: grad_aux must be fp32 [3]")
    out = torch.empty_like(logits)
    st = nat.load().nt_moe_router_bwd(ptr(logits), ptr(ids), ptr(weights), ptr(grad_w),
                                      ptr(counts), T, E, k, score_fn, ptr(grad_aux),
                                      float(aux_coeff), float(z_coeff), ptr(out),
                                      _stream(logits.device))
    nat.check(st, "ntmoe::router_bwd")
    return out


@router_bwd.register_fake
def _(logits, ids, weights, grad_w, counts, score_fn, grad_aux, aux_coeff, z_coeff):
    return torch.empty_like(logits)


@_custom_op("ntmoe::grouped_wgrad")
def grouped_wgrad(a: Tensor, b: Tensor, b_src_row: Optional[Tensor], seg_offsets: Tensor,
                  total_rows: int, splits: int = 1, out_fp32: bool = False) -> Tensor:
    """c [S, N, M]: c[s] = sum over segment s's rows r of a[r]^T b[row(r)], bf16 (or fp32 with
    out_fp32); with splits > 1 each segment's rows run as `splits` chunks whose fp32 sums are
    added in ascending order (for long segments)."""
    _on_gpu(a, b, b_src_row, seg_offsets)
    _require(a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and a.dim() == 2
             and b.dim() == 2 and a.stride(1) == 1 and b.stride(1) == 1,
             "grouped_wgrad: a and b must be bf16 matrices with contiguous rows")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.dim() == 1
             and seg_offsets.is_contiguous(), "grouped_wgrad: seg_offsets must be int32 [S+1]")
    if b_src_row is not None:
        _require(b_src_row.dtype == torch.int32 and b_src_row.is_contiguous(),
                 "grouped_wgrad: b_src_row must be contiguous int32")
    S = seg_offsets.shape[0] - 1
    N, M = a.shape[1], b.shape[1]
    c = torch.empty(S, N, M, device=a.device, dtype=torch.float32 if out_fp32 else torch.bfloat16)
    partial = None
    if splits > 1:
        partial = torch.empty(splits, S, N, M, device=a.device, dtype=torch.float32)
    st = nat.load().nt_moe_grouped_wgrad_splitk(
        ptr(a), a.stride(0), ptr(b), b.stride(0), b.shape[0], ptr(b_src_row), ptr(seg_offsets),
        S, total_rows, N, M, splits, ptr(partial),
        0 if partial is None else partial.numel() * 4, int(out_fp32), ptr(c), _stream(a.device))
    nat.check(st, "ntmoe::grouped_wgrad")
    return c


@grouped_wgrad.register_fake
def _(a, b, b_src_row, seg_offsets, total_rows, splits=1, out_fp32=False):
    return a.new_empty(seg_offsets.shape[0] - 1, a.shape[1], b.shape[1],
                       dtype=torch.float32 if out_fp32 else torch.bfloat16)


@_custom_op("ntmoe::grouped_wgrad_pair")
def grouped_wgrad_pair(a0: Tensor, b0: Tensor, b_src_row0: Optional[Tensor], a1: Tensor,
                       b1: Tensor, b_src_row1: Optional[Tensor], seg_offsets: Tensor,
                       total_rows: int, out_fp32: bool = False) -> tuple[Tensor, Tensor]:
    """(grouped_wgrad(a0, b0, b_src_row0, ...), grouped_wgrad(a1, b1, b_src_row1, ...)) over the
    same segments without split K, bit for bit; one launch when both take the 256 x 256 kernel
    (widths multiples of 256)."""
    _on_gpu(a0, b0, b_src_row0, a1, b1, b_src_row1, seg_offsets)
    for a, b, src in ((a0, b0, b_src_row0), (a1, b1, b_src_row1)):
        _require(a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and a.dim() == 2
                 and b.dim() == 2 and a.stride(1) == 1 and b.stride(1) == 1,
                 "grouped_wgrad_pair: a and b must be bf16 matrices with contiguous rows")
        if src is not None:
            _require(src.dtype == torch.int32 and src.is_contiguous(),
                     "grouped_wgrad_pair: b_src_row must be contiguous int32")
    _require(seg_offsets.dtype == torch.int32 and seg_offsets.dim() == 1
             and seg_offsets.is_contiguous(),
             "grouped_wgrad_pair: seg_offsets must be int32 [S+1]")
    S = seg_offsets.shape[0] - 1
    dt = torch.float32 if out_fp32 else torch.bfloat16
    c0 = torch.empty(S, a0.shape[1], b0.shape[1], device=a0.device, dtype=dt)
    c1 = torch.empty(S, a1.shape[1], b1.shape[1], device=a0.device, dtype=dt)
    st = nat.load().nt_moe_grouped_wgrad_pair(
        ptr(a0), a0.stride(0), ptr(b0), b0.stride(0), b0.shape[0], ptr(b_src_row0), a0.shape[1],
        b0.shape[1], ptr(c0), ptr(a1), a1.stride(0), ptr(b1), b1.stride(0), b1.shape[0],
        ptr(b_src_row1), a1.shape[1], b1.shape[1], ptr(c1), ptr(seg_offsets), S, total_rows,
        int(out_fp32), _stream(a0.device))
    nat.check(st, "ntmoe::grouped_wgrad_pair")
    return c0, c1


@grouped_wgrad_pair.register_fake
def _(a0, b0, b_src_row0, a1, b1, b_src_row1, seg_offsets, total_rows, out_fp32=False):
    S = seg_offsets.shape[0] - 1
    dt = torch.float32 if out_fp32 else torch.bfloat16
    return (a0.new_empty(S, a0.shape[1], b0.shape[1], dtype=dt),
            a0.new_empty(S, a1.shape[1], b1.shape[1], dtype=dt))


_CU_COUNT = {}


def wgrad_splits(segments, N, M, rows_per_segment, device):
    """Chunks per segment for grouped_wgrad: enough workgroups for about two per CU when the
    tiles alone are fewer, each chunk at least 4 slabs (256 rows) long, at most 32."""
    cus = _CU_COUNT.get(device)
    if cus is None:
        cus = _CU_COUNT.setdefault(device, torch.cuda.get_device_properties(device).multi_processor_count)
    tiles = segments * -(-N // 128) * -(-M // 128)
    if tiles >= 2 * cus:
        return 1
    return max(1, min(32, -(-2 * cus // tiles), rows_per_segment // 256))


def split_bf16(t):
    """(hi, lo) bf16 with hi + lo = t to within 2^-17 |t| (hi = t rounded to bf16, lo = the
    remainder, exact in fp32, rounded to bf16): fp32 products on bf16 matrix cores as
    hi.b + lo.b (b exact in bf16), or hi.h + hi.l + lo.h with both operands split."""
    hi = t.to(torch.bfloat16)
    return hi, (t - hi.float()).to(torch.bfloat16)


def _round_up(n, m):
    return (n + m - 1) // m * m


class Projection:
    """One dgrad / recompute GEMM's weights, c[r] = a_r . W_s^T with W [S, n, K] bf16: packed for
    the packed GEMM when the shape qualifies, else the plain grouped GEMM's operand."""

    def __init__(self, w, prepacked=None):
        if prepacked is not None:  # already in the packed layout (convert_pack_expert_weights)
            self.packed, self.w = True, prepacked
            return
        S, n, K = w.shape
        self.packed = prefers_packed(K, n, nat.EPI_NONE)
        self.w = pack_expert_weights.raw(w.contiguous(), nat.EPI_NONE) if self.packed else w.contiguous()

    def __call__(self, a, src_row, seg_offsets, total_rows):
        gemm = grouped_gemm_packed.raw if self.packed else grouped_gemm.raw
        return gemm(a, src_row, seg_offsets, self.w, nat.EPI_NONE, total_rows)


class BackwardWeights:
    """The backward's GEMM operands, built from the bf16 weights the forward used (plain
    layout) and the fp32 router weight, each on first use:
      w1t, w2t     W1^T and W2^T (dgrad of the two projections)
      w1           W1 (recompute of the fc1 pre-activations; only when the forward kept none)
      shared       the shared expert's W2^T (its dgrad)
      shared_w1_proj  the shared expert's W1 (its fc1 recompute; only when the forward kept none)
      first        the token-side first row's operand: [W1s^T | Wr_hi^T | Wr_lo^T | Wr_hi^T]
                   (K padded to 64), so that one GEMM over [dfc1s | g_hi | g_hi | g_lo] gives the
                   shared expert's input gradient plus grad_logits . Wr in fp32 (the router's
                   input gradient; g = grad_logits, hi/lo its two-term bf16 split, hi + lo
                   within about 2^-17 |g| of g) rounded once
    """

    def __init__(self, w1, w2, shared_w1=None, shared_w2=None, w_router_t=None, w1_t=None,
                 w2_t=None, shared_w2_t=None, w1_t_packed=None, w2_t_packed=None,
                 shared_w2_t_packed=None, first=None):
        self.w1_plain, self.w2_plain = w1, w2
        self.shared_w1, self.shared_w2 = shared_w1, shared_w2
        self.w_router_t = w_router_t

        def plain_shape(plain, *transposed):  # [S, rows, cols] of the weight the forward used
            if plain is not None:
                return tuple(plain.shape)
            t = next((t for t in transposed if t is not None), None)
            return None if t is None else (t.shape[0], t.shape[2], t.shape[1])
        # the weight gradients' shapes (what an empty batch returns zeros of)
        self.shapes = dict(w1=plain_shape(w1, w1_t, w1_t_packed),
                           w2=plain_shape(w2, w2_t, w2_t_packed),
                           shared_w1=plain_shape(shared_w1),
                           shared_w2=plain_shape(shared_w2, shared_w2_t, shared_w2_t_packed))
        # transposes already made (convert_expert_weights), else made here on first use
        self._t = dict(w1=w1_t, w2=w2_t, shared_w2=shared_w2_t)
        # transposes already packed (convert_pack_expert_weights), used as they are
        self._tp = dict(w1=w1_t_packed, w2=w2_t_packed, shared_w2=shared_w2_t_packed)
        self._cache = {}
        if first is not None:  # already built with w_router_t (router_operands)
            Fs = 0 if shared_w1 is None else shared_w1.shape[1]
            self._cache["first"] = (first, (Fs,) + first_layout(w_router_t.shape[1], Fs))

    def _transposed(self, name, w):
        t = self._t.get(name)
        return t if t is not None else w.transpose(1, 2).contiguous()

    def _projection_t(self, name, w):
        """The dgrad projection over w^T: from its packed form when given, else from w^T."""
        tp = self._tp.get(name)
        return Projection(None, tp) if tp is not None else Projection(self._transposed(name, w))

    def _get(self, name, make):
        if name not in self._cache:
            self._cache[name] = make()
        return self._cache[name]

    @property
    def w1(self):
        return self._get("w1", lambda: Projection(self.w1_plain))

    @property
    def w1t(self):
        return self._get("w1t", lambda: self._projection_t("w1", self.w1_plain))

    @property
    def w2t(self):
        return self._get("w2t", lambda: self._projection_t("w2", self.w2_plain))

    @property
    def shared(self):
        if self.shared_w1 is None:
            return None
        return self._get("shared", lambda: dict(
            w2t=self._projection_t("shared_w2", self.shared_w2)))

    @property
    def shared_w1_proj(self):
        return self._get("shared_w1", lambda: Projection(self.shared_w1))

    def first(self, w_router_t):
        """[1, d, Kc] bf16 (see the class notes) and the column layout (Fs, Ep, Kc)."""
        def make():
            d, E = w_router_t.shape
            Fs = 0 if self.shared_w1 is None else self.shared_w1.shape[1]
            Ep, Kc = first_layout(E, Fs)
            w = torch.zeros(1, d, Kc, device=w_router_t.device, dtype=torch.bfloat16)
            if Fs:
                w[0, :, :Fs] = self.shared_w1[0].t()
            hi, lo = split_bf16(w_router_t)
            w[0, :, Fs:Fs + E] = hi
            w[0, :, Fs + Ep:Fs + Ep + E] = lo
            w[0, :, Fs + 2 * Ep:Fs + 2 * Ep + E] = hi
            return w, (Fs, Ep, Kc)
        return self._get("first", make)


def backward_weights(w1, w2, shared_w1=None, shared_w2=None, w_router_t=None, **transposes):
    """The backward's GEMM operands (BackwardWeights) from the bf16 weights the forward used
    (and, optionally, their transposes w1_t, w2_t, shared_w2_t)."""
    return BackwardWeights(w1, w2, shared_w1, shared_w2, w_router_t, **transposes)


_unit_cache = {}


def _unit_weights(T, k, device):
    """Cached fp32 ones [T, k] (the unit combine weights of the input-gradient sum), read only;
    a fill kernel less per backward. Holds the last few shapes."""
    key = (T, k, device)
    t = _unit_cache.get(key)
    if t is None:
        if len(_unit_cache) >= 8:
            _unit_cache.clear()
        t = _unit_cache[key] = torch.ones(T, k, device=device, dtype=torch.float32)
    return t


def moe_backward(grad_out, grad_aux, x, w_router_t, bw, state, *, top_k,
                 score_fn=nat.SCORE_SOFTMAX, activation=nat.ACT_SWIGLU, aux_coeff=0.01,
                 z_coeff=0.001, mark=None, weight_grads_fp32=False):
    """Gradients of moe_forward (bf16 experts) for grad_out [T, d] and grad_aux [3] (or None).

    state: moe_forward's state from a call with want_logits=True and keep=True; bw: from
    backward_weights. Returns dict(x bf16 [T, d], router fp32 [E, d] (the router weight's, i.e.
    of w_router_t^T), w1 [E, F, d], w2 [E, d, H], shared_w1, shared_w2 (bf16, or fp32 from the
    same fp32 sums with weight_grads_fp32)). Widths d, F, H (and the shared expert's) must be
    multiples of 64.

    All on this library's kernels: the fc1 recompute (when the forward kept no pre-activations),
    the dgrad of both projections (grouped GEMMs), the combine transpose and routing-weight
    gradient, the activation backward, the router backward (routing-weight, load-balance and
    z-loss terms), the token-side sum of the k input-gradient rows (the forward's combine kernel
    with unit weights; its first row, the shared expert's input gradient plus the router's,
    grad_logits . Wr, comes from one grouped GEMM over the concatenated K of BackwardWeights'
    `first` operand), and every weight gradient on grouped_wgrad: dy^T h and d_fc1^T x over each
    expert's rows (x gathered through src_row), the shared expert's over all T rows and the
    router's grad_logits^T x (fp32 output over the two-term bf16 split of grad_logits, which
    carries g to about 2^-17 |g|; the router gradients are checked against fp64), the last
    two split along T in fixed order. `mark(name)` as in moe_forward.
    """
    mark = mark or (lambda name: None)
    T, d = x.shape
    E = w_router_t.shape[1]
    k = top_k
    A = T * k
    sh = bw.shared_w1 is not None
    if T == 0:  # no rows: every gradient is zero
        wdt = torch.float32 if weight_grads_fp32 else torch.bfloat16
        z = lambda shape: None if shape is None else torch.zeros(shape, device=x.device, dtype=wdt)
        return dict(x=torch.zeros_like(x), router=torch.zeros(E, d, device=x.device),
                    w1=z(bw.shapes["w1"]), w2=z(bw.shapes["w2"]),
                    shared_w1=z(bw.shapes["shared_w1"]), shared_w2=z(bw.shapes["shared_w2"]))
    src, offsets = state["src_row"], state["offsets"]
    cdest, ids = state["combine_dest"], state["ids"]
    g = grad_out.to(torch.bfloat16).contiguous()
    fc1 = state.get("fc1")
    if fc1 is None:  # not kept by the forward: recompute the pre-activations
        fc1 = bw.w1(x, src, offsets, A)
    mark("fc1_recompute")
    gy, gw = combine_bwd.raw(g, state["y"], ids, cdest, state["combine_w"])
    mark("combine_bwd")
    dh = bw.w2t(gy, None, offsets, A)
    mark("dgrad_down")
    dfc1 = act_bwd.raw(fc1, dh, activation)
    mark("act_bwd")
    dxp = bw.w1t(dfc1, None, offsets, A)
    mark("dgrad_up")
    res = dict(shared_w1=None, shared_w2=None)
    seg = _whole_batch_segment(T, x.device)
    dfc1s = None
    if sh:
        sb = bw.shared
        fc1s = state.get("shared_fc1")
        if fc1s is None:  # not kept by the forward
            fc1s = bw.shared_w1_proj(x, None, seg, T)
        dhs = sb["w2t"](g, None, seg, T)
        dfc1s = act_bwd.raw(fc1s, dhs, activation)
        mark("shared")
    dlogits = router_bwd.raw(state["logits"], ids, state["weights"], gw, state["counts"], score_fn,
                         grad_aux, aux_coeff, z_coeff)
    # the token-side first row: [dfc1s | g_hi | g_hi | g_lo] . [W1s^T | Wr_hi | Wr_lo | Wr_hi]^T
    wf, (Fs, Ep, Kc) = bw.first(w_router_t)
    a_cat = backward_first_operand.raw(dlogits, dfc1s, Ep, Kc)
    first = grouped_gemm.raw(a_cat, None, seg, wf, nat.EPI_NONE, T)
    # dWr = grad_logits^T x in fp32: [g_hi | g_lo]^T x (x exact in bf16), fp32 sums split along
    # T; [g_hi | g_lo] are a_cat's last two blocks
    g_cat = a_cat[:, Fs + Ep:Fs + 3 * Ep]
    wr = grouped_wgrad.raw(g_cat, x, None, seg, T, wgrad_splits(1, 2 * Ep, d, T, x.device), True)[0]
    res["router"] = wr[:E] + wr[Ep:Ep + E]
    mark("router_bwd")
    res["x"], _ = combine_aux.raw(dxp, cdest, _unit_weights(T, k, x.device), first,
                                  state["prob_partial"], state["z_partial"], state["counts"],
                                  0.0, 0.0)
    mark("dx_sum")
    # expert weight gradients over each expert's rows; the shared expert's over all T rows
    f32 = weight_grads_fp32
    h = state["h"]
    s1 = wgrad_splits(E, dfc1.shape[1], d, A // E, x.device)
    s2 = wgrad_splits(E, d, h.shape[1], A // E, x.device)
    if s1 == 1 and s2 == 1:  # both in one call (one launch where both take the 256-wide tiles)
        res["w1"], res["w2"] = grouped_wgrad_pair.raw(dfc1, x, src, gy, h, None, offsets, A, f32)
    else:
        res["w1"] = grouped_wgrad.raw(dfc1, x, src, offsets, A, s1, f32)
        res["w2"] = grouped_wgrad.raw(gy, h, None, offsets, A, s2, f32)
    if sh:
        res["shared_w1"] = grouped_wgrad.raw(dfc1s, x, None, seg, T,
                                         wgrad_splits(1, dfc1s.shape[1], d, T, x.device), f32)
        res["shared_w2"] = grouped_wgrad.raw(g, state["shared_h"], None, seg, T,
                                         wgrad_splits(1, d, state["shared_h"].shape[1], T,
                                                      x.device), f32)
    mark("wgrad")
    return res
