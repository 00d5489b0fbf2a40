"""The public backward at the shapes where the backends switch forms, against the fp64 oracle.

``backends.backward`` picks, by batch x heads and chunk count, among the affine-step
recurrences (few heads), the forward scan beside the segmented state recurrence (few heads,
long rows), the paired direct recurrences at 32-wide tiles (17 <= B*H <= 32), 64-wide ones
(up to B*H = 127, with the vector gates' in-kernel qg / kg / w) or 16-wide ones (B*H <= 16 on
short rows), and the fused forward sweep or the plain direct recurrences (B*H >= 128).  One case on each side of each switch, odd head counts
included, every family, both KDA policies: every (batch row, head) pair is independent end to
end, so two heads of each batch (the first and the last) are checked against the oracle run
on that head alone, at the reference's acceptance tolerances (validation.py:40-45, :68).  The
final-state gradient is given, and every family except GDN2 has an initial state."""
import pytest
import torch

from oracle import delta_oracle as O
from tests._inputs import make_inputs

pytestmark = pytest.mark.gpu

OPNAME = {"kda": "chunk_kda", "gdn": "chunk_gated_delta_rule", "gdn2": "chunk_gdn2", "delta": "chunk_delta_rule"}
GRAD = {"q": "dq", "k": "dk", "v": "dv", "g": "dg", "beta": "dbeta", "b": "db", "w": "dw", "initial_state": "dh0"}
CASES = [  # op, B, T, H, full saving
    ("kda", 2, 256, 12, False),       # B*H = 24: paired, 32-wide, kg read by the scan
    ("delta", 1, 512, 20, False),     # 20: paired, 32-wide
    ("gdn2", 1, 256, 17, False),      # 17: paired, 32-wide
    ("gdn2", 1, 256, 33, False),      # 33: paired, 64-wide, qg / kg / w formed in both
    ("gdn", 1, 256, 33, False),       # 33: paired, 64-wide, Aqk in the state recurrence
    ("delta", 1, 256, 65, False),     # 65: paired, 64-wide (130 work-groups a launch)
    ("kda", 1, 256, 65, False),       # 65: paired, 64-wide, vector gate
    ("gdn", 1, 256, 127, False),      # 127: paired, 64-wide (254 work-groups a launch)
    ("gdn2", 2, 256, 64, False),      # 128: one after the other
    ("gdn2", 4, 256, 16, False),      # 64: paired, 64-wide, prepare-free
    ("kda", 4, 256, 16, True),        # full saving at 64
    ("kda", 1, 1024, 4, True),        # full saving, 4 heads, 16 chunks: the direct state recurrence
    ("gdn2", 1, 1088, 4, True),       # full saving, 4 heads, 17 chunks: affine-step
    ("kda", 1, 6144, 16, True),       # full saving, 16 heads, 96 chunks: segmented
    ("kda", 1, 6080, 16, True),       # ... 95 chunks: affine-step
    ("kda", 1, 6144, 24, True),       # full saving, 24 heads, 96 chunks: segmented
    ("gdn2", 1, 6080, 24, True),      # ... 95 chunks: direct
    ("kda", 1, 8192, 8, True),        # full saving, 8 heads, 128 chunks: segmented
    ("gdn2", 1, 12288, 4, True),      # full saving, 4 heads, 192 chunks: segmented
    ("kda", 1, 12224, 4, True),       # ... 191 chunks: affine-step
    ("gdn2", 1, 16384, 47, True),     # full saving, 47 heads, 256 chunks: segmented
    ("kda", 1, 16384, 48, True),      # ... 48 heads: direct
    ("gdn", 1, 1024, 8, False),       # 8 heads, 16 chunks
    ("kda", 1, 4096, 4, False),       # 4 heads, 64 chunks: affine-step or segmented
    ("gdn2", 1, 2048, 16, False),     # 16 heads, 32 chunks: paired, 16-wide
    ("delta", 1, 4096, 16, False),    # 16 heads, 64 chunks: paired, 16-wide
    ("gdn", 1, 8192, 16, False),      # 16 heads, 128 chunks: paired, 16-wide
    ("gdn", 1, 8256, 16, False),      # 16 heads, 129 chunks: the scan beside the segmented recurrence
    ("kda", 2, 512, 8, False),        # B*H = 16, 8 chunks: paired, 16-wide, vector gate
    ("kda", 1, 1024, 15, False),      # 15 heads, 16 chunks: paired, 16-wide
    ("kda", 1, 2048, 8, False),       # 8 heads, 32 chunks: affine-step
    ("delta", 1, 256, 2, False),      # configs[0], 4 chunks: paired, 16-wide
    ("gdn2", 1, 576, 4, False),       # 4 heads, 9 chunks: affine-step
    ("gdn2", 1, 128, 1, False),       # one head, 2 chunks: paired, 16-wide
    ("gdn", 1, 2048, 12, False),      # 12 heads, 32 chunks: paired, 16-wide
    ("delta", 1, 2112, 12, False),    # 12 heads, 33 chunks: paired, 16-wide
    ("delta", 1, 2112, 11, False),    # 11 heads, 33 chunks: affine-step
    ("delta", 8, 256, 16, False),     # 128: the fused sweep
    ("kda", 8, 256, 16, False),       # 128, vector gate
]


@pytest.mark.parametrize("op,B,T,H,full", CASES)
def test_backward_at_policy_boundaries_matches_oracle(op, B, T, H, full):
    import rewy_amd as fdr
    print(f"\n[policy-boundary] op={op} B={B} T={T} H={H} full_saving={full}", flush=True)
    xs, dO = make_inputs(op, B, T, H, seed=1000 + B * 100 + H, gate="mild" if op in ("kda", "gdn2") else "default",
                         h0=op != "gdn2")
    dev = torch.device("cuda")
    leaves = {n: v.to(dev).requires_grad_() for n, v in xs.items()}
    kw = dict(disable_recompute=full) if op in ("kda", "gdn2") else {}
    with fdr.use_backend("optimized", ops=(op,)):
        o, ht = getattr(fdr, OPNAME[op])(**leaves, output_final_state=True, **kw)
    dht = torch.randn(ht.shape, generator=torch.Generator().manual_seed(7)) * 0.05
    grads = dict(zip(leaves, torch.autograd.grad((o, ht), list(leaves.values()), (dO.to(dev), dht.to(dev)))))
    torch.cuda.synchronize()
    fdr.assert_used((op,))
    for bb, hh in ((0, 0), (B - 1, H - 1)):
        def head(x, name):
            if x is None:
                return None
            x = x.detach()
            x = x[bb:bb + 1, hh:hh + 1] if name in ("initial_state", "dht") else x[bb:bb + 1, :, hh:hh + 1]
            return x.double().cpu().numpy()
        ref = O.backward(op, head(xs["q"], "q"), head(xs["k"], "k"), head(xs["v"], "v"),
                         g=head(xs.get("g"), "g"), beta=head(xs.get("beta"), "beta"), b=head(xs.get("b"), "b"),
                         w=head(xs.get("w"), "w"), h0=head(xs.get("initial_state"), "initial_state"),
                         dO=head(dO, "dO"), dht=head(dht, "dht"))
        report = {}
        for name, gr in grads.items():
            e = O.error(ref[GRAD[name]], head(gr, name), O.limit_for(GRAD[name]))
            report[name] = round(e["relative_l2"], 5)
            assert e["passed"], (op, B, T, H, full, (bb, hh), name, e)
        print(f"head ({bb}, {hh}) rel-L2 vs fp64 oracle", report, flush=True)
