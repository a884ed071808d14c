"""Writes the committed fixtures under tests/golden/ (run from the repository root).

    python tests/golden/make_golden.py [--t3 PATH_TO_REFERENCE_t3.json]

moe_small.npz -- routing and forward vectors of the CPU oracle for three small layers whose
    inputs are stored with them (bf16 hidden states and expert weights as raw uint16, fp32
    router and bias): the GPU path is checked against these bit for bit (routing) and within
    the bf16 tolerance (outputs); the oracle is checked against them for drift. Case "ties"
    duplicates router rows, so whole columns of logits tie and the lower-index rule decides.
t3_expert_cells.json -- the data the reference's T3 scaling manifest holds for its expert
    families (configs/scaling/t3.json): top-level keys, expert family recipes, expert cells.
    Only written when --t3 names the manifest.
"""
import argparse
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import moe_oracle as orc  # noqa: E402

CASES = [
    # name, T, d, E, k, H, score_fn, activation, shared_H, bias, seed
    ("ties", 96, 64, 8, 2, 64, orc.SOFTMAX, orc.SWIGLU, 0, False, 100),
    ("sigmoid-relu2-shared-bias", 80, 192, 4, 3, 64, orc.SIGMOID, orc.RELU2, 64, True, 101),
    ("k-equals-E", 5, 64, 4, 4, 64, orc.SOFTMAX, orc.SWIGLU, 0, False, 102),
]


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def make_case(name, T, d, E, k, H, score_fn, activation, shared_H, with_bias, seed):
    g = torch.Generator().manual_seed(seed)
    F = 2 * H if activation == orc.SWIGLU else H
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    router = torch.randn(E, d, generator=g) * 0.02
    if name == "ties":
        router[5] = router[3]
        router[7] = router[0]
    w1 = (torch.randn(E, F, d, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, d, H, generator=g) * 0.02).to(torch.bfloat16)
    out = dict(x=bf16_bits(x), router=router.numpy(), w1=bf16_bits(w1), w2=bf16_bits(w2),
               meta=np.array([T, d, E, k, H, score_fn, activation, shared_H], dtype=np.int64))
    sw1 = sw2 = bias = None
    if shared_H:
        Fs = 2 * shared_H if activation == orc.SWIGLU else shared_H
        sw1 = (torch.randn(Fs, d, generator=g) * 0.02).to(torch.bfloat16)
        sw2 = (torch.randn(d, shared_H, generator=g) * 0.02).to(torch.bfloat16)
        out.update(shared_w1=bf16_bits(sw1), shared_w2=bf16_bits(sw2))
    if with_bias:
        bias = torch.randn(E, generator=g)
        out.update(bias=bias.numpy())
    weights = orc.Weights(router=router, w1=w1.float(), w2=w2.float(),
                          shared_w1=None if sw1 is None else sw1.float(),
                          shared_w2=None if sw2 is None else sw2.float(), bias=bias)
    ref = orc.moe_forward(x, weights, k, score_fn=score_fn, activation=activation)
    for key in ("logits", "ids", "weights", "counts", "offsets", "src_row", "dest", "out"):
        out["ref_" + key] = ref[key].numpy()
    out["ref_aux"] = np.array([ref["aux"], ref["lb"], ref["z"]], dtype=np.float64)
    return {f"{name}/{key}": v for key, v in out.items()}


def write_t3(path):
    data = json.loads(Path(path).read_text())
    experts = ("moe", "looped", "kda-dsa")
    keep = {k: v for k, v in data.items() if not isinstance(v, (list, dict))}
    keep["families"] = [dict(id=f["id"], recipe=f["recipe"]) for f in data["families"]
                        if f["id"] in experts]
    keep["cells"] = [c for c in data["cells"] if c["family"] in experts]
    (HERE / "t3_expert_cells.json").write_text(json.dumps(keep, indent=1, ensure_ascii=False) + "\n")


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--t3", help="path of the reference's configs/scaling/t3.json")
    args = p.parse_args()
    arrays = {}
    for case in CASES:
        arrays.update(make_case(*case))
    np.savez_compressed(HERE / "moe_small.npz", **arrays)
    if args.t3:
        write_t3(args.t3)


if __name__ == "__main__":
    main()
