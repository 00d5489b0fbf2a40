"""Write the per-family golden vectors tests/golden/family_<op>.npz.

Inputs are the seeded BASELINE.json-style tensors of tests/_inputs.py at
B=1, T=128 (two chunks), H=1, K=V=128 with beta zero on every 5th token
(scalar-beta families); bf16 tensors are stored as their uint16 bit patterns.
Outputs are the fp64 oracle's gradients (rounded to fp32) of
<o, dO> + <S_T, dht>.  Run from the repository root:
    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import delta_oracle as O  # noqa: E402
from tests._inputs import make_inputs  # noqa: E402

BF16 = ("q", "k", "v", "b", "w", "dO")


def make(op):
    xs, dO = make_inputs(op, 1, 128, 1, seed=2024, beta_zero_every=5 if op != "gdn2" else 0)
    dht = torch.randn(1, 1, 128, 128, generator=torch.Generator().manual_seed(77)) * 0.1
    n = lambda x: None if x is None else x.double().numpy()
    ref = O.backward(op, n(xs["q"]), n(xs["k"]), n(xs["v"]), g=n(xs.get("g")), beta=n(xs.get("beta")),
                     b=n(xs.get("b")), w=n(xs.get("w")), h0=n(xs["initial_state"]), dO=n(dO), dht=n(dht))
    out = {}
    for name, x in list(xs.items()) + [("dO", dO), ("dht", dht)]:
        if name in BF16:
            out["in_" + name] = x.view(torch.int16).numpy().view(np.uint16)
        else:
            out["in_" + name] = x.float().numpy()
    for name in ("dq", "dk", "dv", "dg", "dbeta", "db", "dw", "dh0"):
        if name in ref:
            out["out_" + name] = ref[name].astype(np.float32)
    out["out_o"] = ref["fwd"]["o"].astype(np.float32)
    out["out_final"] = ref["fwd"]["final"].astype(np.float32)
    np.savez_compressed(Path(__file__).with_name(f"family_{op}.npz"), **out)


def load(op):
    """Inputs as torch tensors (bf16 restored) and expected outputs as numpy."""
    with np.load(Path(__file__).with_name(f"family_{op}.npz"), allow_pickle=False) as d:
        data = {k: d[k] for k in d.files}
    ins, outs = {}, {}
    for k, v in data.items():
        if k.startswith("in_"):
            name = k[3:]
            t = torch.from_numpy(v.copy())
            ins[name] = t.view(torch.bfloat16) if v.dtype == np.uint16 else t
        else:
            outs[k[4:]] = v
    return ins, outs


if __name__ == "__main__":
    for op in O.FAMILIES:
        make(op)
        print("wrote", op)
