"""HIP graph capture of the whole layer forward (torch.cuda.CUDAGraph over the ntmoe ops).

The library allocates nothing, clears nothing with memset and never synchronises; the route plan
and the GEMMs' tile lists are built on the device. So one layer forward captures into a graph,
and every replay must equal an eager forward on the same input, bit for bit. Between replays the
test runs eager forwards (the program's own work) and synchronises.
"""
import pytest
import torch

from tests.moe_cases import Case, make_inputs

pytestmark = pytest.mark.gpu

CASES = [
    (Case("graph-T4096-d1024-E32-k4", 4096, 1024, 32, 4, 512, seed=11), False),
    (Case("graph-T1000-d512-E64-k8-sigmoid-shared", 1000, 512, 64, 8, 256, score_fn=1,
          shared_H=512, zipf_bias=1.2, seed=12), False),
    (Case("graph-fp8-T64-d1024-E32-k4", 64, 1024, 32, 4, 512, seed=13), True),
]


def _weights(case, fp8):
    from nexttransformer_amd import _native as nat, ops
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
    g = dict(wt=cpu["router"].t().contiguous().to(dev),
             logit_bias=None if cpu["bias"] is None else cpu["bias"].to(dev))
    for name, epi in (("w1", up), ("w2", nat.EPI_NONE), ("shared_w1", up),
                      ("shared_w2", nat.EPI_NONE)):
        g[name], g[name + "_scale"] = None, None
        if cpu[name] is None:
            continue
        if fp8:
            q, s = ops.quantize_fp8_blockwise(cpu[name].to(dev))
            g[name], g[name + "_scale"] = ops.pack_expert_weights_fp8(q, epi), s
        else:
            g[name] = ops.pack_expert_weights(cpu[name].to(torch.bfloat16).to(dev), epi)
    return cpu, g


@pytest.mark.parametrize("case,fp8", CASES, ids=[c.name for c, _ in CASES])
def test_layer_forward_replays_from_a_hip_graph(case, fp8):
    from nexttransformer_amd import ops
    cpu, g = _weights(case, fp8)
    wt = g.pop("wt")

    def fwd(x):
        return ops.moe_forward(x, wt, g["w1"], g["w2"], top_k=case.k, score_fn=case.score_fn,
                               activation=case.activation, logit_bias=g["logit_bias"],
                               shared_w1=g["shared_w1"], shared_w2=g["shared_w2"],
                               w1_scale=g["w1_scale"], w2_scale=g["w2_scale"],
                               shared_w1_scale=g["shared_w1_scale"],
                               shared_w2_scale=g["shared_w2_scale"], packed=True)

    gen = torch.Generator().manual_seed(case.seed + 100)
    inputs = [cpu["x"]] + [torch.randn(case.T, case.d, generator=gen).to(torch.bfloat16)
                           for _ in range(3)]
    inputs = [t.cuda() for t in inputs]
    x_static = inputs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as capture requires
        fwd(x_static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, aux, _ = fwd(x_static)
    for rep in range(2):
        for x in inputs:
            x_static.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            ref_out, ref_aux, _ = fwd(x)
            torch.cuda.synchronize()
            assert torch.equal(out, ref_out), f"replay {rep}: output differs from eager"
            assert torch.equal(aux, ref_aux), f"replay {rep}: aux losses differ from eager"
