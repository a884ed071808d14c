"""GPU parity of the plain-weight grouped GEMM's 256 x 256-tile kernel (both operands staged
through LDS; the kernel behind nt_moe_grouped_gemm_bf16 when K >= 128 and n_out % 8 == 0;
n_out = 36 checks the entry point's other kernel) against an fp64
product, over ragged segments (empty, one row, exact, several tiles), gathered and direct rows,
widths that leave partial N tiles (n_out not a multiple of 32), and K from two steps up; and
bit-identity with the packed-weight kernel, which multiplies in the same K order.
Bar: relative L2 1e-2 (bf16 outputs, fp32 accumulation)."""
import numpy as np
import pytest
import torch

from tests.moe_cases import rel_l2
from tests.test_gpu_packed import _ref_gemm

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


@pytest.mark.parametrize("K", [128, 320, 1280])
@pytest.mark.parametrize("epilogue,n_out", [(0, 192), (1, 104), (2, 224), (2, 40), (2, 36)],
                         ids=["swiglu-192", "relu2-104", "plain-224", "plain-40", "plain-36"])
@pytest.mark.parametrize("gather", [False, True])
def test_t256_gemm_matches_fp64(K, epilogue, n_out, gather):
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(3 * K + epilogue + n_out)
    counts = [0, 300, 1, 256, 0, 513, 40, 129]
    S = len(counts)
    R = 2 * n_out if epilogue == 0 else n_out
    rows = sum(counts)
    seg = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    a_rows = 700 if gather else rows
    a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16)
    src = torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32) if gather else None
    w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16)
    print(f"[t256] K={K} epi={epilogue} n_out={n_out} gather={gather}", flush=True)
    c = ops.grouped_gemm(a.cuda(), None if src is None else src.cuda(), seg.cuda(), w.cuda(),
                         epilogue, rows)
    torch.cuda.synchronize()
    assert c.shape == (rows, n_out)
    assert rel_l2(c.float(), _ref_gemm(a, src, seg, w, epilogue)) <= BF16_TOL


@pytest.mark.parametrize("epilogue", [0, 2], ids=["swiglu", "plain"])
def test_t256_many_tiles_and_bit_identical_to_packed(epilogue):
    """More tiles than workgroups (several rounds of the persistent schedule); the output equals
    the packed-weight kernel's bit for bit and sampled rows match fp64."""
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(11 + epilogue)
    K, n_out = 1024, 512
    counts = [9000, 0, 7777, 129, 12000, 1, 6500, 4200]
    S = len(counts)
    R = 2 * n_out if epilogue == 0 else n_out
    rows = sum(counts)
    seg = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    a_rows = 20000
    a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16).cuda()
    src = torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32).cuda()
    w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
    print(f"[t256] many tiles epi={epilogue} rows={rows}", flush=True)
    c = ops.grouped_gemm(a, src, seg.cuda(), w, epilogue, rows)
    cp = ops.grouped_gemm_packed(a, src, seg.cuda(), ops.pack_expert_weights(w, epilogue),
                                 epilogue, rows)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), cp.view(torch.int16))
    pick = torch.randint(0, rows, (300,), generator=g)
    seg_of = torch.searchsorted(seg[1:].long(), pick, right=True)
    a_c, src_c, w_c = a.cpu(), src.cpu(), w.cpu()
    ref = torch.empty(len(pick), n_out, dtype=torch.float64)
    for s_ in range(S):
        m = seg_of == s_
        if m.any():
            z = a_c[src_c[pick[m]].long()].double() @ w_c[s_].double().t()
            ref[m] = torch.nn.functional.silu(z[:, :n_out]) * z[:, n_out:] if epilogue == 0 else z
    assert rel_l2(c.cpu()[pick].float(), ref) <= BF16_TOL
