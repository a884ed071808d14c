"""Loads the committed golden fixtures (tests/golden/moe_small.npz) into torch tensors."""
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "moe_small.npz"


def _bf16(a):
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


def load_golden():
    """name -> dict(x bf16 [T, d], weights (oracle.Weights with bf16-valued fp32 tensors),
    bf16 tensors w1/w2/shared_w1/shared_w2, k, score_fn, activation, ref_* expected values)."""
    from oracle import moe_oracle as orc
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({key.split("/")[0] for key in z.files})
    out = {}
    for name in names:
        get = lambda key: z[f"{name}/{key}"] if f"{name}/{key}" in z.files else None
        T, d, E, k, H, score_fn, activation, shared_H = (int(v) for v in get("meta"))
        case = dict(T=T, d=d, E=E, k=k, H=H, score_fn=score_fn, activation=activation,
                    shared_H=shared_H, x=_bf16(get("x")).reshape(T, d),
                    router=torch.from_numpy(get("router").copy()),
                    w1=_bf16(get("w1")), w2=_bf16(get("w2")),
                    shared_w1=None if get("shared_w1") is None else _bf16(get("shared_w1")),
                    shared_w2=None if get("shared_w2") is None else _bf16(get("shared_w2")),
                    bias=None if get("bias") is None else torch.from_numpy(get("bias").copy()))
        case["weights"] = orc.Weights(
            router=case["router"], w1=case["w1"].float(), w2=case["w2"].float(),
            shared_w1=None if case["shared_w1"] is None else case["shared_w1"].float(),
            shared_w2=None if case["shared_w2"] is None else case["shared_w2"].float(),
            bias=case["bias"])
        for key in ("logits", "ids", "weights", "counts", "offsets", "src_row", "dest", "out"):
            case["ref_" + key] = torch.from_numpy(get("ref_" + key).copy())
        case["ref_aux"] = get("ref_aux")
        out[name] = case
    return out
