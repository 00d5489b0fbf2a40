"""Benchmark of the chunked delta-rule backward on one MI355X.

Default workload: KDA (per-channel gate) chunk backward with full saving at
B=8, T=4096, H=16, K=V=128, chunk 64 -- BASELINE.json configs[2], the
configuration the headline metric names.  One "step" is one complete backward
(state recurrence kernel + fused chunk kernel) over synthetic inputs already
resident in HBM; the forward that produces the saved tensors runs once,
outside the timed region.

Printed (one JSON line): backward ms per step, algorithmic TFLOP/s and its
fraction of the bf16 MFMA peak, a roofline record for the dominant kernel
(per-launch algorithmic bytes / HIP-event launch time), the same-GPU time of
the original 7-product formulation (PyTorch ops) and a CPU baseline (the fp64
oracle on a bounded sample, one thread).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "delta-rule bwd ms + TFLOP/s (frac of MFMA peak), KDA/GDN B=8 T=4096 H=16"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

# per chunk-head (64 tokens x one head), K = V = 128 -- see DESIGN.md
CONFIGS = {
    "kda": dict(op="kda", B=8, T=4096, H=16, seed=2, gate="kda", h0=False, full_saving=True),
    "kda_long": dict(op="kda", B=1, T=65536, H=16, seed=4, gate="kda_long", h0=True, full_saving=True),
}
FLOP_STATE = 2 * (64 * 128 * 128 + 64 * 64 * 128 + 2 * 128 * 64 * 128)          # 7.34 MFLOP
FLOP_CHUNK = 2 * (3 * 64 * 64 * 128 + 3 * 64 * 128 * 128 + 4 * 64 * 64 * 128)   # 13.63 MFLOP
BYTES_STATE = 3 * 16384 + 16384 + 16384 + 512 + 32768 + 16384                   # qg,kg,w,dO,Aqk,g_last | dh,dR
BYTES_CHUNK = (5 * 16384 + 32768 + 256 + 16384 + 2 * 32768) + (3 * 16384 + 32768 + 256)


def make_inputs(cfg, device):
    import torch
    import torch.nn.functional as F
    B, T, H, K = cfg["B"], cfg["T"], cfg["H"], 128
    gen = torch.Generator().manual_seed(cfg["seed"])
    shape = (B, T, H, K)
    q = F.normalize(torch.randn(shape, generator=gen), dim=-1).bfloat16()
    k = F.normalize(torch.randn(shape, generator=gen), dim=-1).bfloat16()
    v = torch.randn(shape, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(shape[:-1], generator=gen))
    if cfg["gate"] == "kda_long":
        g = F.logsigmoid(0.3 * torch.randn(shape, generator=gen) + 3)
    else:
        g = F.logsigmoid(torch.randn(shape, generator=gen)).clamp_min(-5)
    h0 = torch.randn(B, H, K, K, generator=gen) * 0.02 if cfg["h0"] else None
    dO = torch.randn(shape, generator=gen).bfloat16()
    dev = lambda x: None if x is None else x.to(device)
    return dict(q=dev(q), k=dev(k), v=dev(v), beta=dev(beta), g=dev(g), h0=dev(h0)), dev(dO)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="kda", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-original", action="store_true", help="skip the torch original comparator")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (reference kernel for the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); every GPU box in this "
              "build has one GPU and the path shards over batch*heads with no exchange.", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        n = 1 << 28                                   # 1 GiB of fp32
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": 4 * n, "calibrate_copy_bytes_written": 4 * n}))
        return
    from rewy_amd import ops
    from rewy_amd.backends.backward import kda_backward
    from rewy_amd.forward import chunk_forward
    from rewy_amd.runtime import check_baseline

    check_baseline()
    cfg = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    xs, dO = make_inputs(cfg, dev)
    B, T, H = cfg["B"], cfg["T"], cfg["H"]
    NTt = B * H * (T // 64)
    print(f"[bench] config={args.config} B={B} T={T} H={H} chunk-heads={NTt}", file=sys.stderr, flush=True)
    with torch.no_grad():
        _, _, sv = chunk_forward("kda", xs["q"], xs["k"], xs["v"], g=xs["g"], beta=xs["beta"],
                                 initial_state=xs["h0"])
    torch.cuda.synchronize()
    scale = sv["scale"]
    dht = None

    def step():
        return kda_backward(q=xs["q"], k=xs["k"], v=xs["v"], beta=xs["beta"], Aqk=sv["Aqk"],
                            Akk=sv["Akk"], scale=scale, initial_state=xs["h0"], do=dO, dht=dht,
                            g=sv["gc"], w=sv["w"], u=sv["u"], qg=sv["qg"], kg=sv["kg"],
                            v_new=sv["v_new"], h=sv["h"], disable_recompute=True)

    # ---- gradient check against the original formulation (same GPU, same inputs) ----
    from rewy_amd.original import original_backward
    got = step()
    torch.cuda.synchronize()
    parity = None
    t_orig = None
    if not args.no_original:
        def orig():
            return original_backward("kda", xs["q"], xs["k"], xs["v"], sv["gc"], sv["Akk"], scale,
                                     xs["h0"], dO, dht, beta=xs["beta"], Aqk=sv["Aqk"], saved=sv)
        ref = orig()
        torch.cuda.synchronize()
        parity = {}
        for name, a, r in (("dq", got[0], ref["dq"]), ("dk", got[1], ref["dk"]), ("dv", got[2], ref["dv"]),
                           ("dbeta", got[3], ref["dbeta"]), ("dg", got[4], ref["dg"])):
            a, r = a.double(), r.double()
            parity[name] = dict(rel_l2=float((a - r).norm() / r.norm().clamp_min(1e-30)),
                                max_abs=float((a - r).abs().max()))
        del ref
        torch.cuda.synchronize()
        n_orig = 3
        t0 = time.perf_counter()
        for _ in range(n_orig):
            orig()
        torch.cuda.synchronize()
        t_orig = (time.perf_counter() - t0) / n_orig * 1e3

    # ---- timed region: complete backward, W warmup + K steps ----
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3

    # ---- per-kernel launch times with HIP events on the launch stream ----
    stream = torch.cuda.current_stream(dev)
    reps = max(5, args.steps)

    def time_kernel(fn):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in evs:
            a.record(stream)
            fn()
            b.record(stream)
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in evs) / reps

    t_state = time_kernel(lambda: ops.state_bwd(sv["qg"], sv["kg"], sv["w"], sv["gc"], ops.GATE_VECTOR, dO,
                                                scale, aqk=sv["Aqk"], dht=dht, want_dh0=xs["h0"] is not None))
    dh, dR, _ = ops.state_bwd(sv["qg"], sv["kg"], sv["w"], sv["gc"], ops.GATE_VECTOR, dO, scale,
                              aqk=sv["Aqk"], dht=dht, want_dh0=False)
    t_chunk = time_kernel(lambda: ops.chunk_bwd(xs["q"], xs["k"], xs["v"], sv["v_new"], dO, dR, sv["gc"],
                                                ops.GATE_VECTOR, sv["Akk"], sv["h"], dh, scale, beta=xs["beta"]))
    kernels = {
        "fdr_state_bwd": dict(ms=t_state, gbs=BYTES_STATE * NTt / (t_state * 1e-3) / 1e9,
                              tflops=FLOP_STATE * NTt / (t_state * 1e-3) / 1e12),
        "fdr_chunk_bwd": dict(ms=t_chunk, gbs=BYTES_CHUNK * NTt / (t_chunk * 1e-3) / 1e9,
                              tflops=FLOP_CHUNK * NTt / (t_chunk * 1e-3) / 1e12),
    }
    dom = max(kernels, key=lambda n: kernels[n]["ms"])
    dom_bytes = (BYTES_CHUNK if dom == "fdr_chunk_bwd" else BYTES_STATE) * NTt
    achieved = kernels[dom]["gbs"]
    flops = (FLOP_STATE + FLOP_CHUNK) * NTt
    tflops = flops / (ms * 1e-3) / 1e12

    # ---- CPU baseline: fp64 oracle of the same two stages on a bounded sample ----
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(xs, sv, dO, dh, dR, scale, NTt)

    line = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (BASELINE.json distributions, seeded)",
        "config": {"workload": f"{cfg['op']} chunk backward, full saving, B={B} T={T} H={H} K=V=128 chunk=64",
                   "global_batch": B, "seq_len": T, "heads": H, "parallelism": "none (1 GPU)"},
        "tflops": round(tflops, 2),
        "mfma_peak_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "kernels": {n: {kk: round(vv, 4) for kk, vv in d.items()} for n, d in kernels.items()},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(dom, args.config), "algorithmic_bytes_per_launch": dom_bytes},
        "original_torch_ms": None if t_orig is None else round(t_orig, 3),
        "speedup_vs_original_torch": None if t_orig is None else round(t_orig / ms, 2),
        "parity_vs_original": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def measured_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/hbm_traffic.json, calibrated against a plain
    copy of known size), or None when that workload was not profiled."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data[config][kernel]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(xs, sv, dO, dh, dR, scale, NTt, heads_per_piece=1):
    """fp64 oracle (numpy, one thread) of the timed stages -- state recurrence and
    chunk stage -- on a bounded sample (batch 0, all T, the first 8 heads, one
    head at a time so the oracle's pairwise tensors stay small), scaled linearly
    to the full workload's chunk-head count."""
    import numpy as np
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    from oracle import delta_oracle as O
    B, T, H = xs["q"].shape[:3]
    heads = H
    nb = min(B, 3)                               # batches 0..nb-1, every head: ~10 s of fp64 work
    sample_heads = nb * heads * (T // 64)
    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    if ctx:
        ctx.__enter__()
    el = 0.0
    try:
        for bb, h0 in [(bb, h0) for bb in range(nb) for h0 in range(0, heads, heads_per_piece)]:
            hs = slice(h0, h0 + heads_per_piece)
            n = lambda x: x[bb:bb + 1, :, hs].double().cpu().numpy()
            inp = dict(qg=n(sv["qg"]), kg=n(sv["kg"]), w=n(sv["w"]), gc=n(sv["gc"]), dO=n(dO),
                       Aqk=n(sv["Aqk"]), q=n(xs["q"]), k=n(xs["k"]), v=n(xs["v"]), beta=n(xs["beta"]),
                       Akk=n(sv["Akk"]), h=n(sv["h"]), v_new=n(sv["v_new"]))
            t0 = time.perf_counter()
            dvl = O.dv_local(inp["Aqk"], inp["dO"])
            d_h, d_R, _ = O.stage_state_bwd(inp["qg"], inp["kg"], inp["w"], inp["gc"], inp["dO"], dvl,
                                            scale=scale)
            O.stage_post("kda", inp["q"], inp["k"], inp["v"], inp["gc"], beta=inp["beta"], Akk=inp["Akk"],
                         h=inp["h"], dh=d_h, v_new=inp["v_new"], dO=inp["dO"], dR=d_R, scale=scale)
            el += time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    full_ms = el * 1e3 * NTt / sample_heads
    return {"value": round(full_ms, 1), "unit": "ms (full workload, extrapolated)", "cores": 1,
            "kind": "port",
            "sample": f"fp64 numpy oracle (state recurrence + chunk stage), batches 0-{nb - 1}, T={T}, all {heads} heads "
                      f"({sample_heads} of {NTt} chunk-heads), measured {el:.2f} s, scaled linearly"}


if __name__ == "__main__":
    main()
