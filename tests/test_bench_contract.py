"""bench.py's contract pieces that need no GPU: the multi-GPU refusal and the
algorithmic cost model (per chunk-head FLOPs and bytes quoted in the design notes,
FLOPs per the residual formulation of the metric's definition)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_kernel_costs_match_the_quoted_figures():
    import bench
    kda = bench.kernel_costs("kda", True)
    assert set(kda) >= {"fdr_state_bwd", "fdr_chunk_bwd"}
    assert kda["fdr_state_bwd"][0] == 131_584 and kda["fdr_chunk_bwd"][0] == 279_040
    # 20.97 MFLOP per chunk-head for KDA with full saving (residual formulation)
    total = kda["fdr_state_bwd"][1] + kda["fdr_chunk_bwd"][1]
    assert total == pytest.approx(20.97e6, rel=1e-3)
    gdn = bench.kernel_costs("gdn", False)
    assert gdn["fdr_prepare_wu"][0] == 115_200 and gdn["fdr_fwd_h"][0] == 98_564
    # the affine-step launches are costed as the recurrences they replace
    assert gdn["affine_recurrences"] == tuple(a + b for a, b in zip(gdn["fdr_fwd_h"], gdn["fdr_state_bwd"]))
    assert kda["affine_state"] == kda["fdr_state_bwd"]
    # Aqk formed in the state recurrence (no Aqk read; q k^T computed there), w / u in the
    # forward scan's sweep: k, v, Akk, g, beta read, w, h, v_new written
    inl = bench.kernel_costs("gdn", False, inline=True)
    assert inl["fdr_fwd_h_wy"][0] == 115_200
    assert inl["fdr_prepare_wu"][0] == gdn["fdr_prepare_wu"][0] - bench.TILE - bench.AT
    assert inl["fdr_state_bwd"][0] == gdn["fdr_state_bwd"][0] - bench.AT
    assert inl["fdr_state_bwd"][1] == gdn["fdr_state_bwd"][1] + 2 * 64 * 64 * 128
    assert bench.inline_aqk(bench.CONFIGS["gdn"]) and not bench.inline_aqk(bench.CONFIGS["kda"])


def test_paper_grid_tables_are_complete():
    import bench
    assert len(bench.PAPER_GRID) == 6
    for (op, policy), (orig, rewy) in bench.H100_US.items():
        assert op in bench.PAPER_GATE and policy in ("recompute", "all")
        assert len(orig) == len(rewy) == 6
        assert all(o > r > 0 for o, r in zip(orig, rewy))     # ReWY beat FLA in every published case


def test_every_config_is_costed_as_its_backward_runs():
    """The cost model of every bench config, with the paired recurrences' in-kernel forms as
    the backend picks them (pure host logic: ``pair_forms`` and ``kernel_costs``)."""
    import bench
    for name, cfg in bench.CONFIGS.items():
        raw, formw = bench.pair_forms(cfg)
        costs = bench.kernel_costs(cfg["op"], cfg["full_saving"], bench.inline_aqk(cfg), bench.folds_u(cfg), raw,
                                   formw)
        assert all(b > 0 and f > 0 for b, f in costs.values()), name
        assert formw <= raw
        assert ("fdr_prepare_wu" in costs) == (not cfg["full_saving"] and not formw), name
    # GDN2 B=2 T=8192 H=32 (64-wide paired tiles): w, qg, kg and u formed in the recurrences
    assert bench.pair_forms(bench.CONFIGS["gdn2"]) == (True, True)
    assert bench.pair_forms(bench.CONFIGS["kda"]) == (False, False)          # full saving
