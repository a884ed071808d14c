"""ctypes binding of libnt_moe.so, the C ABI declared in include/nt_moe.h.

The library is built in-tree by `nexttransformer_amd.build` (or `__graft_entry__.build()`).
There is no fallback: if the library is missing, every op raises.
"""
import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libnt_moe.so"

NT_MOE_OK = 0
NT_MOE_EINVAL = -22
NT_MOE_ENOSPC = -28
NT_MOE_EDEVICE = -5
ABI_VERSION = 1

SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1
ACT_SWIGLU, ACT_RELU2 = 0, 1
EPI_SWIGLU, EPI_RELU2, EPI_NONE = 0, 1, 2
MAX_EXPERTS, MAX_TOPK, MAX_SEGMENTS, ROUTE_BLOCK = 256, 8, 512, 64
NOALLOC_MAX_ASSIGNMENTS = NOALLOC_MAX_BLOCK_COUNTS = 1 << 18

_p, _i64, _i32, _f32, _sz = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
                             ctypes.c_size_t)

# name -> (restype, argtypes); the order follows include/nt_moe.h.
SIGNATURES = {
    "nt_moe_abi_version": (_i32, []),
    "nt_moe_last_error": (ctypes.c_char_p, []),
    "nt_moe_router_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32]),
    "nt_moe_router_fwd": (_i32, [_p, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p,
                                 _p, _p, _sz, _p]),
    "nt_moe_topk_from_logits": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _p]),
    "nt_moe_route_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "nt_moe_histogram_scan": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p, _sz, _p]),
    "nt_moe_permute": (_i32, [_p, _i64, _p, _p, _i64, _i32, _i32, _i32, _p, _sz, _p, _p, _p, _p,
                              _p, _p]),
    "nt_moe_route_plan": (_i32, [_p, _i64, _p, _p, _i64, _i32, _i32, _i32, _p, _p, _p, _sz, _p,
                                 _p, _p, _p, _p, _p]),
    "nt_moe_router_plan_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32]),
    "nt_moe_router_plan": (_i32, [_p, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p,
                                  _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "nt_moe_route_plan_noalloc": (_i32, [_p, _i64, _p, _p, _i64, _i32, _i32, _i32, _p, _p, _p,
                                         _p, _p, _p, _p, _p]),
    "nt_moe_grouped_gemm_bf16_packed_keep": (_i32, [_p, _i64, _i64, _p, _p, _i32, _i64, _p, _i32,
                                                    _i32, _i32, _p, _p, _p]),
    "nt_moe_grouped_wgrad_bf16": (_i32, [_p, _i64, _p, _i64, _i64, _p, _p, _i32, _i64, _i32, _i32,
                                         _p, _p]),
    "nt_moe_grouped_wgrad_splitk": (_i32, [_p, _i64, _p, _i64, _i64, _p, _p, _i32, _i64, _i32,
                                           _i32, _i32, _p, _sz, _i32, _p, _p]),
    "nt_moe_combine_bwd": (_i32, [_p, _i64, _p, _p, _p, _p, _i64, _i32, _i32, _p, _p, _p]),
    "nt_moe_act_bwd": (_i32, [_p, _p, _i64, _i32, _i32, _p, _p]),
    "nt_moe_router_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _p, _f32, _f32, _p,
                                 _p]),
    "nt_moe_grouped_gemm_workspace_bytes": (_sz, []),
    "nt_moe_grouped_ffn_bf16": (_i32, [_p, _i64, _i64, _p, _p, _i32, _i64, _p, _p, _i32, _i32,
                                       _i32, _p, _p, _p, _sz, _p]),
    "nt_moe_grouped_gemm_bf16": (_i32, [_p, _i64, _i64, _p, _p, _i32, _i64, _p, _i32, _i32, _i32,
                                        _p, _p, _sz, _p]),
    "nt_moe_grouped_gemm_bf16_keep": (_i32, [_p, _i64, _i64, _p, _p, _i32, _i64, _p, _i32, _i32,
                                             _i32, _p, _p, _p]),
    "nt_moe_convert_expert_weights": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p]),
    "nt_moe_convert_expert_weights_packed": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p, _i32, _p,
                                                    _p]),
    "nt_moe_grouped_wgrad_pair": (_i32, [_p, _i64, _p, _i64, _i64, _p, _i32, _i32, _p, _p, _i64,
                                          _p, _i64, _i64, _p, _i32, _i32, _p, _p, _i32, _i64,
                                          _i32, _p]),
    "nt_moe_router_operands": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _i64, _i32, _p, _p, _i32,
                                       _i32, _p]),
    "nt_moe_pack_expert_weights_bf16": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _p]),
    "nt_moe_grouped_gemm_bf16_packed": (_i32, [_p, _i64, _i64, _p, _p, _i32, _i64, _p, _i32, _i32,
                                               _i32, _p, _p]),
    "nt_moe_quantize_fp8_rowwise": (_i32, [_p, _i64, _i64, _i32, _p, _i64, _p, _p]),
    "nt_moe_quantize_fp8_blockwise": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p]),
    "nt_moe_grouped_gemm_fp8": (_i32, [_p, _i64, _i64, _p, _p, _p, _i32, _i64, _p, _p, _i32, _i32,
                                       _i32, _p, _p]),
    "nt_moe_pack_expert_weights_fp8": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _p]),
    "nt_moe_grouped_gemm_fp8_packed": (_i32, [_p, _i64, _i64, _p, _p, _p, _i32, _i64, _p, _p, _i32,
                                              _i32, _i32, _p, _p]),
    "nt_moe_combine_aux": (_i32, [_p, _p, _p, _i64, _i32, _i32, _p, _i64, _p, _i64, _p, _p, _p,
                                  _i32, _f32, _f32, _p, _p]),
    "nt_moe_backward_first_operand": (_i32, [_p, _i32, _p, _i32, _i64, _i32, _i32, _p, _p]),
}

_LIB = None


class NativeLibraryMissing(RuntimeError):
    pass


def load():
    """The loaded library (cached). Raises NativeLibraryMissing when it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise NativeLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -m nexttransformer_amd.build` "
            "(the MoE ops have no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.nt_moe_abi_version() != ABI_VERSION:
        raise NativeLibraryMissing(f"{LIB_PATH}: ABI {lib.nt_moe_abi_version()} != {ABI_VERSION}")
    _LIB = lib
    return lib


def check(status, what):
    """Map an NT_MOE status to the reference's exception types (ValueError / RuntimeError)."""
    if status == NT_MOE_OK:
        return
    message = load().nt_moe_last_error().decode(errors="replace")
    if status in (NT_MOE_EINVAL, NT_MOE_ENOSPC):
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what}: status {status}: {message}")


def ptr(tensor):
    """Device address of a tensor, or None (NULL) for None."""
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())
