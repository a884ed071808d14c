"""GPU parity of the fp8 path (OCP e4m3fn) against the CPU oracle.

Bar: quantisation codes and scales bit-exact (byte work); the fp8 grouped GEMM within relative
L2 1e-2 of the fp32 product of the same dequantised operands (only accumulation order and the
bf16 output rounding differ); the fp8 layer within relative L2 3e-2 of the oracle's fp32
dequantised reference (oracle.moe_forward_fp8), routing bit-exact.
"""
import pytest
import torch

from oracle import moe_oracle as orc
from tests.moe_cases import CONFIGS, rel_l2

pytestmark = pytest.mark.gpu

FP8_LAYER_TOL = 3e-2
FP8_GEMM_TOL = 1e-2


def _mixed_rows(T, d, seed):
    """bf16 rows spanning many binades, an all-zero row and a one-hot row."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g) * torch.exp2(torch.randint(-8, 9, (T, 1), generator=g)).float()
    if T > 2:
        x[1] = 0
        x[2] = 0
        x[2, 5] = -3.0
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("T,d", [(1, 32), (37, 4096), (300, 1536)])
def test_rowwise_quantisation_bit_exact(T, d):
    from nexttransformer_amd import ops
    x = _mixed_rows(T, d, T)
    q, s = ops.quantize_fp8_rowwise(x.cuda())
    ref_q, ref_s = orc.quantize_rowwise(x.float())
    assert torch.equal(s.cpu(), ref_s)
    assert torch.equal(q.cpu(), ref_q)


def test_blockwise_quantisation_bit_exact():
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(3)
    w = torch.randn(3, 256, 384, generator=g) * 0.02
    w[1, :128, :128] = 0
    w[2, 128:, 256:] *= 1e-3
    q, s = ops.quantize_fp8_blockwise(w.cuda())
    ref_q, ref_s = orc.quantize_blockwise(w)
    assert torch.equal(s.cpu(), ref_s)
    assert torch.equal(q.cpu(), ref_q)


def _segments(counts):
    off = [0]
    for c in counts:
        off.append(off[-1] + c)
    return torch.tensor(off, dtype=torch.int32)


@pytest.mark.parametrize("epilogue", [0, 1, 2], ids=["swiglu", "relu2", "none"])
def test_fp8_pack_layout(epilogue):
    """Packed fp8 layout against its definition, rebuilt on the CPU with numpy indexing."""
    import numpy as np
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(20 + epilogue)
    S, R, K = 2, 256, 384
    n_out = R // 2 if epilogue == 0 else R
    w = torch.randint(0, 256, (S, R, K), generator=g, dtype=torch.uint8)
    got = ops.pack_expert_weights_fp8(w.cuda(), epilogue).cpu().numpy().reshape(-1, 16)
    wn = w.numpy()
    NB, KB = R // 32, K // 128
    lanes = np.arange(64)
    i = lanes % 32
    want = np.empty((S, NB, KB, 2, 2, 64, 16), dtype=np.uint8)
    for nb in range(NB):
        rows = np.where(i < 16, 16 * nb + i, n_out + 16 * nb + i - 16) if epilogue == 0 else 32 * nb + i
        for kb in range(KB):
            for st in range(2):
                for h in range(2):
                    k0 = kb * 128 + st * 64 + 32 * (lanes // 32) + 16 * h
                    want[:, nb, kb, st, h] = wn[:, rows[:, None], k0[:, None] + np.arange(16)[None, :]]
    assert np.array_equal(got, want.reshape(-1, 16))


@pytest.mark.parametrize("epilogue", [0, 1, 2], ids=["swiglu", "relu2", "none"])
@pytest.mark.parametrize("gather", [False, True])
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_fp8_grouped_gemm_matches_dequantised_product(epilogue, gather, packed):
    from nexttransformer_amd import _native as nat
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(10 + epilogue)
    counts = [0, 5, 1, 33, 0, 70, 2]  # empty, short, longer than one 32-row chunk
    S, K, n_out = len(counts), 512, 256
    R = 2 * n_out if epilogue == nat.EPI_SWIGLU else n_out
    rows = sum(counts)
    src = torch.randint(0, 50, (rows,), generator=g, dtype=torch.int32) if gather else None
    a_rows = 50 if gather else rows
    a = _mixed_rows(a_rows, K, 5)
    w = torch.randn(S, R, K, generator=g) * 0.05
    aq, as_ = orc.quantize_rowwise(a.float())
    wq, ws = orc.quantize_blockwise(w)
    seg = _segments(counts)
    wdev = ops.pack_expert_weights_fp8(wq.cuda(), epilogue) if packed else wq.cuda()
    c = ops.grouped_gemm_fp8(aq.cuda(), as_.cuda(), None if src is None else src.cuda(),
                             seg.cuda(), wdev, ws.cuda(), epilogue, rows, packed)
    torch.cuda.synchronize()
    a_deq = orc.dequantize_rowwise(aq, as_).double()
    w_deq = orc.dequantize_blockwise(wq, ws).double()
    ref = torch.zeros(rows, n_out, dtype=torch.float64)
    for s_ in range(S):
        lo, hi = int(seg[s_]), int(seg[s_ + 1])
        if hi == lo:
            continue
        idx = src[lo:hi].long() if gather else torch.arange(lo, hi)
        z = a_deq[idx] @ w_deq[s_].t()
        if epilogue == nat.EPI_SWIGLU:
            z = torch.nn.functional.silu(z[:, :n_out]) * z[:, n_out:]
        elif epilogue == nat.EPI_RELU2:
            z = torch.relu(z).square()
        ref[lo:hi] = z
    assert rel_l2(c.float(), ref) <= FP8_GEMM_TOL


def _fp8_layer_inputs(T, d, E, H, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(T, d, generator=g, device=device).to(torch.bfloat16)
    router = torch.randn(E, d, generator=g, device=device) * 0.02
    w1 = torch.randn(E, 2 * H, d, generator=g, device=device) * 0.02
    w2 = torch.randn(E, d, H, generator=g, device=device) * 0.02
    return x, router, w1, w2


@pytest.mark.parametrize("T,d,E,k,H", [(64, 512, 16, 4, 256), (5, 256, 8, 8, 128),
                                         (200, 1024, 32, 2, 512)])
@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_fp8_layer_matches_dequantised_reference(T, d, E, k, H, packed):
    from nexttransformer_amd import ops
    x, router, w1, w2 = _fp8_layer_inputs(T, d, E, H, T + d, "cpu")
    w1q, w1s = ops.quantize_fp8_blockwise(w1.cuda())
    w2q, w2s = ops.quantize_fp8_blockwise(w2.cuda())
    pk = (lambda t, e: ops.pack_expert_weights_fp8(t, e)) if packed else (lambda t, e: t)
    out, aux, st = ops.moe_forward(x.cuda(), router.t().contiguous().cuda(), pk(w1q, 0),
                                   pk(w2q, 2), top_k=k, w1_scale=w1s, w2_scale=w2s,
                                   packed=packed)
    torch.cuda.synchronize()
    ref = orc.moe_forward_fp8(x, router, w1q.cpu(), w1s.cpu(), w2q.cpu(), w2s.cpu(), k)
    assert torch.equal(st["ids"].cpu(), ref["ids"])
    assert torch.equal(st["counts"].cpu(), ref["counts"])
    assert torch.equal(st["x_q"].cpu(), ref["x_q"])
    assert rel_l2(out.float(), ref["out"]) <= FP8_LAYER_TOL
    assert aux[0].item() == pytest.approx(ref["aux"], rel=1e-5)


def test_fp8_layer_config5_full_size():
    """Config 5 at its real size (T=64, d=4096, E=128, k=8, H=1536): routing for every token,
    outputs of sampled tokens against the dequantised reference."""
    from nexttransformer_amd import ops
    case = CONFIGS[5]
    x, router, w1, w2 = _fp8_layer_inputs(case.T, case.d, case.E, case.H, 5, "cuda")
    w1q, w1s = ops.quantize_fp8_blockwise(w1)
    del w1
    w2q, w2s = ops.quantize_fp8_blockwise(w2)
    del w2
    out, aux, st = ops.moe_forward(x, router.t().contiguous(),
                                   ops.pack_expert_weights_fp8(w1q, 0),
                                   ops.pack_expert_weights_fp8(w2q, 2), top_k=case.k,
                                   w1_scale=w1s, w2_scale=w2s, packed=True)
    torch.cuda.synchronize()
    tokens = [0, 17, 40, 63]
    ref = orc.moe_forward_fp8(x.cpu(), router.cpu(), w1q, w1s, w2q, w2s, case.k, tokens=tokens)
    assert torch.equal(st["ids"].cpu(), ref["ids"])
    assert torch.equal(st["counts"].cpu(), ref["counts"])
    assert int(st["counts"].sum()) == case.T * case.k
    assert rel_l2(out[tokens].float(), ref["out"]) <= FP8_LAYER_TOL
