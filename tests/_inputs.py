"""Seeded synthetic inputs shared by the tests (BASELINE.json distributions)."""
import torch
import torch.nn.functional as F


def make_inputs(op, B, T, H, K=128, seed=0, gate="default", h0=True, beta_zero_every=0):
    g_ = torch.Generator().manual_seed(seed)
    shape = (B, T, H, K)
    q = F.normalize(torch.randn(shape, generator=g_), dim=-1).bfloat16()
    k = F.normalize(torch.randn(shape, generator=g_), dim=-1).bfloat16()
    v = torch.randn(shape, generator=g_).bfloat16()
    xs = dict(q=q, k=k, v=v)
    if op == "gdn2":
        xs["b"] = (torch.rand(shape, generator=g_) * 0.8 + 0.1).bfloat16()
        xs["w"] = (torch.rand(shape, generator=g_) * 0.8 + 0.1).bfloat16()
    else:
        beta = torch.sigmoid(torch.randn(shape[:-1], generator=g_))
        if beta_zero_every:
            beta[:, ::beta_zero_every] = 0.0
        xs["beta"] = beta
    if op == "gdn":
        xs["g"] = F.logsigmoid(torch.randn(shape[:-1], generator=g_) * 0.5 + 4)
    elif op in ("kda", "gdn2"):
        if gate == "wide":
            xs["g"] = F.logsigmoid(torch.randn(shape, generator=g_) * 3 - 4)
        elif gate == "mild":      # long-memory gates (BASELINE.json's kda_long draw)
            xs["g"] = F.logsigmoid(torch.randn(shape, generator=g_) * 0.3 + 3)
        else:
            xs["g"] = F.logsigmoid(torch.randn(shape, generator=g_)).clamp_min(-5)
    if h0:
        xs["initial_state"] = torch.randn(B, H, K, K, generator=g_) * 0.02
    dO = torch.randn(B, T, H, K, generator=g_).bfloat16()
    return xs, dO
