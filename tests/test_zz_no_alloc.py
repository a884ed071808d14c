"""GPU check of nt_moe_route_plan_noalloc (the route plan whose scratch is a static device array
of the library) against nt_moe_route_plan (the same plan with a caller workspace), called
through the C ABI: two calls in a row, the second with a smaller input (so the static scratch
holds the first call's data), plus one with the row gather (x_perm), all bit-exact; sizes
beyond the static limits are rejected before anything is launched."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _routing(T, E, k, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    w = torch.rand(T, k, generator=g)
    return ids.cuda(), (w / w.sum(1, keepdim=True)).cuda()


def _outputs(T, E, k, d, want_x):
    dev = torch.device("cuda")
    i32, f32 = torch.int32, torch.float32
    return dict(counts=torch.full((E,), -7, dtype=i32, device=dev),
                offsets=torch.full((E + 1,), -7, dtype=i32, device=dev),
                src=torch.full((T * k,), -7, dtype=i32, device=dev),
                perm_w=torch.full((T * k,), -7.0, dtype=f32, device=dev),
                dest=torch.full((T, k), -7, dtype=i32, device=dev),
                cw=torch.full((T, k), -7.0, dtype=f32, device=dev),
                x_perm=torch.zeros(T * k, d, dtype=torch.bfloat16, device=dev) if want_x else None)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _plan(lib, ids, w, E, x, noalloc):
    from nexttransformer_amd import _native as nat
    T, k = ids.shape
    d = 0 if x is None else x.shape[1]
    o = _outputs(T, E, k, d, x is not None)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        st = lib.nt_moe_route_plan_noalloc(_p(x), 0 if x is None else x.stride(0), _p(ids), _p(w),
                                           T, d, k, E, _p(o["counts"]), _p(o["offsets"]),
                                           _p(o["src"]), _p(o["perm_w"]), _p(o["dest"]),
                                           _p(o["cw"]), _p(o["x_perm"]), stream)
    else:
        nbytes = lib.nt_moe_route_workspace_bytes(T, k, E)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        st = lib.nt_moe_route_plan(_p(x), 0 if x is None else x.stride(0), _p(ids), _p(w), T, d,
                                   k, E, _p(o["counts"]), _p(o["offsets"]), _p(ws), nbytes,
                                   _p(o["src"]), _p(o["perm_w"]), _p(o["dest"]), _p(o["cw"]),
                                   _p(o["x_perm"]), stream)
    nat.check(st, "route_plan_noalloc" if noalloc else "route_plan")
    torch.cuda.synchronize()
    return o


def _assert_same(a, b):
    for name in a:
        if a[name] is None:
            continue
        x, y = a[name], b[name]
        if x.dtype == torch.float32:
            x, y = x.view(torch.int32), y.view(torch.int32)
        elif x.dtype == torch.bfloat16:
            x, y = x.view(torch.int16), y.view(torch.int16)
        assert torch.equal(x, y), name


def test_route_plan_noalloc_matches_route_plan():
    from nexttransformer_amd import _native as nat
    lib = nat.load()
    cases = [(32768, 128, 8, None, 1),   # the largest benchmark plan: T k = 2^18
             (3000, 32, 4, None, 2),     # smaller: the scratch still holds the call above
             (700, 16, 2, 64, 3)]        # with the row gather (histogram + scan + permute)
    for T, E, k, d, seed in cases:
        print(f"[noalloc] T={T} E={E} k={k} x_perm={d is not None}", flush=True)
        ids, w = _routing(T, E, k, seed)
        x = None
        if d is not None:
            x = torch.randn(T, d, generator=torch.Generator().manual_seed(seed)).to(
                torch.bfloat16).cuda()
        got = _plan(lib, ids, w, E, x, noalloc=True)
        want = _plan(lib, ids, w, E, x, noalloc=False)
        _assert_same(got, want)
        assert int(got["counts"].sum()) == T * k
        assert torch.equal(got["counts"].cpu(),
                           torch.bincount(ids.flatten().long().cpu(), minlength=E).to(torch.int32))


def test_route_plan_noalloc_rejects_sizes_beyond_its_scratch():
    from nexttransformer_amd import _native as nat
    lib = nat.load()
    ids, w = _routing(8, 16, 2, 4)
    dummy = torch.empty(16, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    T_big = nat.NOALLOC_MAX_ASSIGNMENTS // 2 + 1  # T k > the limit at k = 2
    st = lib.nt_moe_route_plan_noalloc(None, 0, _p(ids), _p(w), T_big, 0, 2, 16, _p(dummy),
                                       _p(dummy), _p(dummy), _p(dummy), _p(dummy), _p(dummy),
                                       None, stream)
    assert st == nat.NT_MOE_EINVAL
    assert b"static scratch" in lib.nt_moe_last_error()
