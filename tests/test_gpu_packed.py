"""GPU parity of the packed-weight grouped GEMM (weights pre-packed in fragment order, streamed
into registers) against an fp32 reference, and of the layer forward that uses it against the
CPU oracle. Bar: relative L2 1e-2 (bf16 outputs, fp32 accumulation in a different K order than
the unpacked kernel); routing bit-exact as everywhere.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.moe_cases import Case, make_inputs, rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _pack_reference(w, epilogue):
    """The documented packed layout, built on the CPU with numpy indexing."""
    S, R, K = w.shape
    n_out = R // 2 if epilogue == 0 else R
    NB, KB = R // 32, K // 64
    wn = w.view(torch.int16).numpy()
    out = np.empty((S, NB, KB, 4, 64, 8), dtype=np.int16)
    lanes = np.arange(64)
    pos = lanes % 32
    # block position p holds logical row p with its middle 4-row groups swapped per 16-row half
    # (positions 4-7 <-> 8-11, 20-23 <-> 24-27), so that accumulator element i of lane half h is
    # logical row 8 (2 (i // 8) + h) + i % 8
    i = np.array([[0, 2, 1, 3][(p % 16) // 4] * 4 + p % 4 + 16 * (p // 16) for p in pos])
    for nb in range(NB):
        rows = np.where(i < 16, 16 * nb + i, n_out + 16 * nb + i - 16) if epilogue == 0 else 32 * nb + i
        for kb in range(KB):
            for q in range(4):
                k0 = kb * 64 + 32 * (lanes // 32) + 8 * q
                cols = k0[:, None] + np.arange(8)[None, :]
                out[:, nb, kb, q] = wn[:, rows[:, None], cols]
    return torch.from_numpy(out.reshape(S, R, K)).view(torch.bfloat16)


@pytest.mark.parametrize("epilogue", [0, 2], ids=["swiglu", "plain"])
def test_pack_layout(epilogue):
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(1)
    w = torch.randn(3, 128, 256, generator=g).to(torch.bfloat16)
    got = ops.pack_expert_weights(w.cuda(), epilogue).cpu()
    assert torch.equal(got.view(torch.int16), _pack_reference(w, epilogue).view(torch.int16))


def _ref_gemm(a, src, seg, w, epilogue):
    rows = int(seg[-1])
    R = w.shape[1]
    n_out = R // 2 if epilogue == 0 else R
    out = torch.zeros(rows, n_out, dtype=torch.float64)
    for s in range(w.shape[0]):
        lo, hi = int(seg[s]), int(seg[s + 1])
        if hi == lo:
            continue
        idx = src[lo:hi].long() if src is not None else torch.arange(lo, hi)
        z = a[idx].double() @ w[s].double().t()
        if epilogue == 0:
            z = torch.nn.functional.silu(z[:, :n_out]) * z[:, n_out:]
        elif epilogue == 1:
            z = torch.relu(z).square()
        out[lo:hi] = z
    return out


# K = 320 and 448 are odd counts of 64-wide K steps (the extra step that multiplies nothing)
@pytest.mark.parametrize("K", [256, 320, 384, 448, 1024])
@pytest.mark.parametrize("epilogue", [0, 1, 2], ids=["swiglu", "relu2", "plain"])
@pytest.mark.parametrize("gather", [False, True])
def test_packed_gemm_matches_fp32(K, epilogue, gather):
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(K + epilogue)
    counts = [0, 300, 1, 256, 0, 513, 40]  # empty, partial, exact, multi-tile segments
    S, n_out = len(counts), 160 if epilogue == 0 else 224  # partial N tiles too
    R = 2 * n_out if epilogue == 0 else n_out
    rows = sum(counts)
    seg = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    a_rows = 700 if gather else rows
    a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16)
    src = torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32) if gather else None
    w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16)
    wp = ops.pack_expert_weights(w.cuda(), epilogue)
    c = ops.grouped_gemm_packed(a.cuda(), None if src is None else src.cuda(), seg.cuda(), wp,
                                epilogue, rows)
    torch.cuda.synchronize()
    assert rel_l2(c.float(), _ref_gemm(a, src, seg, w, epilogue)) <= BF16_TOL


@pytest.mark.parametrize("K", [512, 1024])
@pytest.mark.parametrize("epilogue", [0, 2], ids=["swiglu", "plain"])
@pytest.mark.parametrize("gather", [False, True])
@pytest.mark.parametrize("rows_scale", [1, 3])
def test_packed_gemm_many_tiles(K, epilogue, gather, rows_scale):
    # Enough tiles for full rounds of the two-workgroups-per-CU schedule plus a last partial
    # round (split into halves or not, by size); every output row must be written, and sampled
    # rows of every segment match fp32.
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(7 * K + epilogue + rows_scale)
    counts = [c * rows_scale for c in [9000, 0, 7777, 129, 12000, 1, 6500, 4200]]
    S, n_out = len(counts), 512
    R = 2 * n_out if epilogue == 0 else n_out
    rows = sum(counts)
    seg = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    a_rows = 20000 if gather else rows
    a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16)
    src = torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32) if gather else None
    w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16)
    wp = ops.pack_expert_weights(w.cuda(), epilogue)
    c = ops.grouped_gemm_packed(a.cuda(), None if src is None else src.cuda(), seg.cuda(), wp,
                                epilogue, rows)
    c2 = ops.grouped_gemm_packed(a.cuda(), None if src is None else src.cuda(), seg.cuda(), wp,
                                 epilogue, rows)
    torch.cuda.synchronize()
    c = c.cpu()
    assert torch.isfinite(c.float()).all() and torch.equal(c, c2.cpu())
    pick = torch.cat([torch.arange(lo, min(lo + 40, hi)) for lo, hi in
                      zip(seg[:-1].tolist(), seg[1:].tolist()) if hi > lo]
                     + [torch.randint(0, rows, (200,), generator=g)])
    a_idx = src[pick].long() if gather else pick
    seg_of = torch.searchsorted(seg[1:].long(), pick, right=True)
    ref = torch.empty(len(pick), n_out, dtype=torch.float64)
    for s_ in range(S):
        m = seg_of == s_
        if m.any():
            z = a[a_idx[m]].double() @ w[s_].double().t()
            ref[m] = torch.nn.functional.silu(z[:, :n_out]) * z[:, n_out:] if epilogue == 0 else z
    assert rel_l2(c[pick].float(), ref) <= BF16_TOL


@pytest.mark.parametrize("epilogue", [1, 2], ids=["relu2", "plain"])
@pytest.mark.parametrize("gather", [False, True])
def test_packed_gemm_t3_widths_many_tiles(epilogue, gather):
    # The registered T3 cell's widths: K = 320 (five K steps per tile) for the down projection,
    # 320 output columns (ten 32-row blocks: the second N tile's last three waves multiply
    # nothing) for the up projection; 256 segments with ragged counts, two launches equal.
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(31 + epilogue + 2 * gather)
    S, K, n_out = 256, 320, 320
    counts = torch.randint(0, 700, (S,), generator=g)
    counts[::17] = 0
    rows = int(counts.sum())
    seg = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).to(torch.int32)
    a_rows = 30000 if gather else rows
    a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16)
    src = torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32) if gather else None
    w = (torch.randn(S, n_out, K, generator=g) * 0.05).to(torch.bfloat16)
    wp = ops.pack_expert_weights(w.cuda(), epilogue)
    args = (a.cuda(), None if src is None else src.cuda(), seg.cuda(), wp, epilogue, rows)
    c = ops.grouped_gemm_packed(*args)
    c2 = ops.grouped_gemm_packed(*args)
    torch.cuda.synchronize()
    c = c.cpu()
    assert torch.isfinite(c.float()).all() and torch.equal(c, c2.cpu())
    pick = torch.cat([torch.arange(lo, min(lo + 8, hi)) for lo, hi in
                      zip(seg[:-1].tolist(), seg[1:].tolist()) if hi > lo]
                     + [torch.randint(0, rows, (300,), generator=g)])
    a_idx = src[pick].long() if gather else pick
    seg_of = torch.searchsorted(seg[1:].long(), pick, right=True)
    ref = torch.empty(len(pick), n_out, dtype=torch.float64)
    for s_ in seg_of.unique().tolist():
        m = seg_of == s_
        z = a[a_idx[m]].double() @ w[s_].double().t()
        ref[m] = torch.relu(z).square() if epilogue == 1 else z
    assert rel_l2(c[pick].float(), ref) <= BF16_TOL


@pytest.mark.parametrize("seed", range(12))
def test_packed_equals_plain_random_shapes(seed):
    # The packed kernel (EDGE instantiation for odd K-step counts and partial N tiles) and the
    # 256 x 256 plain-weight kernel add each output's products in the same K order, so their
    # outputs are equal bit for bit: random K (multiple of 64, >= 256), widths, segment counts.
    from nexttransformer_amd import ops
    g = torch.Generator().manual_seed(1000 + seed)
    epilogue = seed % 3
    K = 64 * int(torch.randint(4, 21, (1,), generator=g))
    n_out = 32 * int(torch.randint(1, 21, (1,), generator=g))
    S = int(torch.randint(1, 40, (1,), generator=g))
    counts = torch.randint(0, 600, (S,), generator=g)
    counts[torch.randint(0, S, (max(1, S // 5),), generator=g)] = 0
    rows = int(counts.sum())
    if rows == 0:
        counts[0], rows = 1, 1
    seg = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).to(torch.int32).cuda()
    R = 2 * n_out if epilogue == 0 else n_out
    gather = seed % 2 == 0
    a_rows = 3000 if gather else rows
    a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16).cuda()
    src = torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32).cuda() if gather else None
    w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
    packed = ops.grouped_gemm_packed(a, src, seg, ops.pack_expert_weights(w, epilogue), epilogue,
                                     rows)
    plain = ops.grouped_gemm(a, src, seg, w, epilogue, rows)
    torch.cuda.synchronize()
    assert torch.equal(packed.view(torch.int16), plain.view(torch.int16)), (K, n_out, S, epilogue)


_EIGHT_WAVE_CHECK = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from nexttransformer_amd import ops
g = torch.Generator().manual_seed(5)
for epilogue, K, n_out in [(0, 1024, 512), (1, 512, 256), (2, 512, 1024)]:
    counts = torch.tensor([700, 0, 1300, 90, 2500])
    seg = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).to(torch.int32).cuda()
    rows = int(counts.sum())
    R = 2 * n_out if epilogue == 0 else n_out
    a = torch.randn(3000, K, generator=g).to(torch.bfloat16).cuda()
    src = torch.randint(0, 3000, (rows,), generator=g, dtype=torch.int32).cuda()
    w = (torch.randn(5, R, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
    p = ops.grouped_gemm_packed(a, src, seg, ops.pack_expert_weights(w, epilogue), epilogue, rows)
    q = ops.grouped_gemm(a, src, seg, w, epilogue, rows)
    torch.cuda.synchronize()
    assert torch.equal(p.view(torch.int16), q.view(torch.int16)), (epilogue, K, n_out)
print("eight-wave ok")
"""


def test_eight_wave_shape_matches_plain():
    # NT_MOE_PACKED_WAVES=8 (read once per process, so in a child process): one 8-wave
    # workgroup per CU with 256-token tiles, its own epilogue transpose geometry (one weight
    # block per wave); outputs equal the plain-weight kernel's bit for bit.
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    env = dict(os.environ, NT_MOE_PACKED_WAVES="8")
    r = subprocess.run([sys.executable, "-c", _EIGHT_WAVE_CHECK, root], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "eight-wave ok" in r.stdout, r.stdout + r.stderr


_PP_CHECK = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from nexttransformer_amd import _native as nat, ops
g = torch.Generator().manual_seed(7)
n = 0
for counts in ([0, 300, 1, 256, 0, 513, 40], [512, 512, 512, 512], [3000, 17, 0, 1200]):
    for K in (256, 320, 1024):
        for epilogue, n_out in ((0, 192), (0, 512), (1, 448), (1, 320), (2, 448), (2, 1024)):
            for gather in (False, True):
                ct = torch.tensor(counts)
                seg = torch.cat([torch.zeros(1, dtype=torch.long), ct.cumsum(0)]).to(torch.int32).cuda()
                rows, S = int(ct.sum()), len(counts)
                R = 2 * n_out if epilogue == 0 else n_out
                a_rows = 3500 if gather else rows
                a = torch.randn(a_rows, K, generator=g).to(torch.bfloat16).cuda()
                src = (torch.randint(0, a_rows, (rows,), generator=g, dtype=torch.int32).cuda()
                       if gather else None)
                w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
                wp = ops.pack_expert_weights(w, epilogue)
                p = ops.grouped_gemm_packed(a, src, seg, wp, epilogue, rows)
                q = ops.grouped_gemm(a, src, seg, w, epilogue, rows)
                torch.cuda.synchronize()
                assert torch.equal(p.view(torch.int16), q.view(torch.int16)), (counts, K, epilogue, n_out, gather)
                if epilogue != 2:  # the fc1 pre-activations equal the plain product's bf16 bits
                    c, pre = ops.grouped_gemm_packed_keep(a, src, seg, wp, epilogue, rows)
                    z = ops.grouped_gemm(a, src, seg, w, nat.EPI_NONE, rows)
                    torch.cuda.synchronize()
                    assert torch.equal(c.view(torch.int16), q.view(torch.int16))
                    assert torch.equal(pre.view(torch.int16), z.view(torch.int16)), (counts, K, epilogue)
                n += 1
print("variant ok", n)
"""


@pytest.mark.parametrize("switch", ["NT_MOE_GEMM_PP"])
def test_256_tile_kernels_match_plain(switch):
    # NT_MOE_GEMM_PP=1 (read once per process, so in a child process): the packed entry points
    # run the two-group ping-pong kernel (256 x 256 tiles, both operands staged in LDS). Its
    # outputs and kept pre-activations equal the plain-weight kernel's bit for bit on empty,
    # single-row, exact and multi-tile segments, partial N tiles (last tiles of 2, 4 and 6 weight
    # blocks), odd K-step counts, with and without the row gather.
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    env = dict(os.environ, **{switch: "1"})
    r = subprocess.run([sys.executable, "-c", _PP_CHECK, root], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "variant ok" in r.stdout, r.stdout + r.stderr


PACKED_CASES = [
    Case("cfg1-shape", 512, 256, 8, 2, 512),
    Case("ragged-T1000-E32-k4", 1000, 1024, 32, 4, 512, seed=1),
    Case("E128-k8-sigmoid", 300, 512, 128, 8, 256, score_fn=1, seed=2),
    Case("relu2-d1280-H384-shared", 130, 1280, 16, 4, 384, activation=1, shared_H=256, seed=4),
    Case("zipf-E64-k8", 777, 256, 64, 8, 256, zipf_bias=1.2, seed=3),
]


@pytest.mark.parametrize("case", PACKED_CASES, ids=lambda c: c.name)
def test_layer_forward_packed_matches_oracle(case):
    from nexttransformer_amd import _native as nat
    from nexttransformer_amd import ops
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
    pk = lambda t, e: None if t is None else ops.pack_expert_weights(t.to(torch.bfloat16).to(dev), e)
    out, aux, st = ops.moe_forward(
        cpu["x"].to(dev), cpu["router"].t().contiguous().to(dev), pk(cpu["w1"], up),
        pk(cpu["w2"], nat.EPI_NONE), top_k=case.k, score_fn=case.score_fn,
        activation=case.activation, logit_bias=None if cpu["bias"] is None else cpu["bias"].to(dev),
        shared_w1=pk(cpu["shared_w1"], up), shared_w2=pk(cpu["shared_w2"], nat.EPI_NONE),
        packed=True)
    torch.cuda.synchronize()
    r = lambda t: None if t is None else t.to(torch.bfloat16).float()
    weights = orc.Weights(router=cpu["router"], w1=r(cpu["w1"]), w2=r(cpu["w2"]),
                          shared_w1=None if cpu["shared_w1"] is None else r(cpu["shared_w1"])[0],
                          shared_w2=None if cpu["shared_w2"] is None else r(cpu["shared_w2"])[0],
                          bias=cpu["bias"])
    ref = orc.moe_forward(cpu["x"], weights, case.k, score_fn=case.score_fn,
                          activation=case.activation)
    assert torch.equal(st["ids"].cpu(), ref["ids"])
    assert torch.equal(st["counts"].cpu(), ref["counts"])
    assert rel_l2(out.float(), ref["out"]) <= BF16_TOL
    assert aux[0].item() == pytest.approx(ref["aux"], rel=1e-4)


def test_packed_forward_is_deterministic():
    from nexttransformer_amd import ops
    case = Case("det", 4096, 1024, 32, 4, 512, seed=13)
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    w1 = ops.pack_expert_weights(cpu["w1"].to(torch.bfloat16).to(dev), 0)
    w2 = ops.pack_expert_weights(cpu["w2"].to(torch.bfloat16).to(dev), 2)
    x, wt = cpu["x"].to(dev), cpu["router"].t().contiguous().to(dev)
    runs = [ops.moe_forward(x, wt, w1, w2, top_k=case.k, packed=True)[:2] for _ in range(3)]
    for out, aux in runs[1:]:
        assert torch.equal(out.view(torch.int16), runs[0][0].view(torch.int16))
        assert torch.equal(aux, runs[0][1])


@pytest.mark.parametrize("epilogue,n_out", [(1, 288), (2, 288), (1, 320)],
                         ids=["relu2-one-block", "plain-one-block", "relu2-two-blocks"])
def test_split_partial_tiles_match_plain(epilogue, n_out):
    """Gathered products whose last N tile holds one or two weight blocks run it split over the
    waves by token block (every wave takes those blocks with its own 32 rows): outputs and the
    kept pre-activations bit for bit equal to the plain-weight kernel's, over segments that end
    inside each wave's rows, with odd and even K-step counts (SwiGLU's split tiles, 160 outputs,
    are checked against fp32 in test_packed_gemm_matches_fp32: the plain kernel takes no SwiGLU
    width that is not a multiple of 64)."""
    from nexttransformer_amd import _native as nat, ops
    for K in (320, 512):
        g = torch.Generator().manual_seed(n_out + K + epilogue)
        counts = torch.tensor([0, 1, 31, 33, 64, 97, 128, 129, 300, 0, 513])
        seg = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).to(torch.int32).cuda()
        rows, S = int(counts.sum()), len(counts)
        R = 2 * n_out if epilogue == 0 else n_out
        a = torch.randn(2000, K, generator=g).to(torch.bfloat16).cuda()
        src = torch.randint(0, 2000, (rows,), generator=g, dtype=torch.int32).cuda()
        w = (torch.randn(S, R, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
        wp = ops.pack_expert_weights(w, epilogue)
        packed = ops.grouped_gemm_packed(a, src, seg, wp, epilogue, rows)
        plain = ops.grouped_gemm(a, src, seg, w, epilogue, rows)
        torch.cuda.synchronize()
        assert torch.equal(packed.view(torch.int16), plain.view(torch.int16)), K
        if epilogue != nat.EPI_NONE:
            c, pre = ops.grouped_gemm_packed_keep(a, src, seg, wp, epilogue, rows)
            z = ops.grouped_gemm(a, src, seg, w, nat.EPI_NONE, rows)
            torch.cuda.synchronize()
            assert torch.equal(c.view(torch.int16), plain.view(torch.int16)), K
            assert torch.equal(pre.view(torch.int16), z.view(torch.int16)), K
