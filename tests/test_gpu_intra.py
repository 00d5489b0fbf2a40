"""The standalone matrix intra seam (fdr_matrix_intra, rewy_amd.backends.intra)
against the fp64 oracle's pairwise intra (oracle.intra_pairwise, itself pinned by
finite differences and by the reference's FLA-captured fixtures).

The comparison is on the intra *increments* (output minus the partial gradient
handed in), so the partials cannot mask an error in the added terms.  The
kernel's contractions split every fp32 operand into bf16 hi + lo (three MFMAs
per product, fp32 accumulation), so the increments match the fp64 oracle to
~1e-5 relative (measured 4e-6 .. 1.5e-5); the tests allow rel-L2 <= 5e-5.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 5e-5


def _rel(a, r):
    return float(np.linalg.norm(a - r) / max(np.linalg.norm(r), 1e-30))


def _run(x, vec, beta_complete=False):
    """x: dict of float64 numpy arrays [B,T,H,*]; returns HIP outputs and oracle outputs."""
    from rewy_amd.backends.intra import chunk_gdn2_bwd_intra, chunk_kda_bwd_intra
    dev = "cuda"
    t = {n: torch.from_numpy(np.ascontiguousarray(v)).float().to(dev) for n, v in x.items()}
    q, k = t["q"].bfloat16(), t["k"].bfloat16()
    parts = [t[n].clone() for n in ("dq", "dk", "db", "dg")]
    ptrs = [p.data_ptr() for p in parts]
    if vec:
        out = chunk_gdn2_bwd_intra(q, k, t["g"], t["b"].bfloat16(), t["dAqk"], t["dAkk"], *parts)
    else:
        out = chunk_kda_bwd_intra(q, k, t["g"], t["beta"], t["dAqk"], t["dAkk"], *parts, beta_complete=beta_complete)
    torch.cuda.synchronize()
    assert [o.data_ptr() for o in out] == ptrs          # in place, like the reference's dq2 = dq
    got = [o.double().cpu().numpy() for o in out]
    qn = q.double().cpu().numpy()
    kn = k.double().cpu().numpy()
    be = t["b"].bfloat16().double().cpu().numpy() if vec else x["beta"]
    # the oracle treats its T axis as one chunk: fold the chunks into the batch axis
    B, T = qn.shape[:2]
    fold = lambda a: a.reshape(B * (T // 64), 64, *a.shape[2:])
    ref = O.intra_pairwise(*(fold(a) for a in (qn, kn, x["g"], be, x["dAqk"], x["dAkk"], x["dq"], x["dk"],
                                                x["db"], x["dg"])), vector_beta=vec)
    ref = [r.reshape(a.shape) for r, a in zip(ref, (x["dq"], x["dk"], x["db"], x["dg"]))]
    if not vec and beta_complete:
        keep = np.abs(x["beta"]) < 1e-6
        ref[2] = x["db"] + np.where(keep, ref[2] - x["db"], 0.0)
    return got, ref


def _check(got, ref, x, label):
    for name, a, r, base in zip(("dq", "dk", "db", "dg"), got, ref, (x["dq"], x["dk"], x["db"], x["dg"])):
        inc_a, inc_r = a - base, r - base
        if np.abs(inc_r).max() == 0:
            assert np.abs(inc_a).max() == 0, (label, name)
            continue
        err = _rel(inc_a, inc_r)
        print(f"{label} {name} increment rel-L2 {err:.2e}", flush=True)
        assert err <= TOL, (label, name, err)


@pytest.mark.parametrize("family", ["kda", "gdn2"])
def test_intra_seam_on_the_reference_captured_fixture(family):
    """validation/npu950_intra/{kda,gdn2}.npz: FLA-captured inputs and pre-intra
    partials (gates reach -138 in log2 units, so most 16-row blocks take the
    exact pairwise diagonal)."""
    meta = json.loads((GOLDEN / "npu950_intra_metadata.json").read_text())[family]
    with np.load(GOLDEN / f"npu950_intra_{family}.npz", allow_pickle=False) as data:
        x = {k: data[k].astype(np.float64) for k in data.files}
    assert meta["dtypes"]["q"] == "torch.bfloat16"
    got, ref = _run(x, family == "gdn2")
    _check(got, ref, x, family)


def _random(vec, B, T, H, seed, gate_scale):
    rng = np.random.default_rng(seed)
    K = 128
    nrm = lambda a: a / np.linalg.norm(a, axis=-1, keepdims=True)
    x = dict(q=nrm(rng.standard_normal((B, T, H, K))), k=nrm(rng.standard_normal((B, T, H, K))))
    raw = np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, K))))) * gate_scale   # logsigmoid
    c = raw.reshape(B, T // 64, 64, H, K).cumsum(2).reshape(B, T, H, K) / np.log(2)
    x["g"] = c.astype(np.float32).astype(np.float64)
    if vec:
        x["b"] = rng.uniform(0.1, 0.9, (B, T, H, K))
    else:
        be = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
        be[:, ::5] = 0.0                                      # rows that take the direct dbeta branch
        x["beta"] = be.astype(np.float32).astype(np.float64)
    x["dAqk"] = (rng.standard_normal((B, T, H, 64)) * 1e-2).astype(np.float32).astype(np.float64)
    x["dAkk"] = (rng.standard_normal((B, T, H, 64)) * 1e-2).astype(np.float32).astype(np.float64)
    # partials of the increments' size, so the fp32 rounding of partial + increment
    # stays far below the tolerance
    for n in ("dq", "dk", "dg"):
        x[n] = (rng.standard_normal((B, T, H, K)) * 1e-3).astype(np.float32).astype(np.float64)
    x["db"] = (rng.standard_normal((B, T, H, K) if vec else (B, T, H)) * 1e-3).astype(np.float32).astype(np.float64)
    return x


@pytest.mark.parametrize("vec", [False, True])
@pytest.mark.parametrize("gate_scale", [1.0, 4.0])
def test_intra_seam_random(vec, gate_scale):
    """Two chunks, three heads; gate_scale 4 makes some 16-row blocks wide enough
    (span >= 80 log2 units) for the pairwise diagonal."""
    x = _random(vec, 2, 128, 3, seed=11 + int(vec), gate_scale=gate_scale)
    blocks = x["g"].reshape(2, 8, 16, 3, 128)
    wide = ((blocks.max(2) - blocks.min(2)) >= 80).mean()
    assert (wide > 0) == (gate_scale > 1), wide             # scale 4 exercises the pairwise diagonal
    got, ref = _run(x, vec)
    _check(got, ref, x, f"vec={vec} scale={gate_scale}")


def test_intra_seam_beta_complete_only_updates_fallback_rows():
    x = _random(False, 1, 128, 2, seed=5, gate_scale=1.0)
    got, ref = _run(x, False, beta_complete=True)
    _check(got, ref, x, "beta_complete")
    keep = np.abs(x["beta"]) >= 1e-6
    np.testing.assert_array_equal(got[2][keep], x["db"][keep].astype(np.float32))
