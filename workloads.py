"""Synthetic inputs for the five benchmark configurations of the Cut Cross-Entropy path.

Every tensor is drawn from a ``torch.Generator`` on the target device, seeded with
the configuration index, in float32 and then rounded to the configuration dtype;
the same call on the same device type always yields the same inputs.

  c1  N=512,   D=512,  V=32000,  fp32, no bias, 5% ignored (26 rows), mean
  c2  [4,1024,2048]  x V=128256, bf16, no bias, 3% ignored (123 rows), mean
  c3  [8,1024,4096]  x V=128256, bf16, Zipf(1.1) targets, peaked e, mean
  c4  [4,1024,2304]  x V=256000, bf16, bias ~ N(0, 0.1^2), 5% ignored (205 rows), none
  c5  [8,4096,8192]  x V=128256, bf16, peaked e, Zipf targets, last 410 of each
      sequence ignored (10%), c ~ N(0, 0.015^2), sum

``scale`` shrinks N (keeps D and V) for parity tests at reduced cost.
"""

import torch

IGNORE = -100

CONFIGS = {
    "c1": dict(B=1, T=512, D=512, V=32000, dtype=torch.float32, c_std=0.02, bias_std=None,
               targets="uniform", ignore_frac=0.05, ignore_count=26, reduction="mean", peaked=False),
    "c2": dict(B=4, T=1024, D=2048, V=128256, dtype=torch.bfloat16, c_std=0.02, bias_std=None,
               targets="uniform", ignore_frac=0.03, ignore_count=123, reduction="mean", peaked=False),
    "c3": dict(B=8, T=1024, D=4096, V=128256, dtype=torch.bfloat16, c_std=0.02, bias_std=None,
               targets="zipf", ignore_frac=0.0, ignore_count=0, reduction="mean", peaked=True),
    "c4": dict(B=4, T=1024, D=2304, V=256000, dtype=torch.bfloat16, c_std=0.02, bias_std=0.1,
               targets="uniform", ignore_frac=0.05, ignore_count=205, reduction="none", peaked=False),
    "c5": dict(B=8, T=4096, D=8192, V=128256, dtype=torch.bfloat16, c_std=0.015, bias_std=None,
               targets="zipf", ignore_frac=0.10, ignore_count=None, pad_tail=410, reduction="sum", peaked=True),
}
NAMES = {
    "c1": "cpu-plumbing N=512 D=512 V=32000 fp32",
    "c2": "Llama-3.2-1B head N=4096 D=2048 V=128256 bf16",
    "c3": "Llama-3.1-8B head N=8192 D=4096 V=128256 bf16",
    "c4": "Gemma-2-2B head+bias N=4096 D=2304 V=256000 bf16",
    "c5": "70B head N=32768 D=8192 V=128256 bf16",
}


def zipf_targets(gen, n, V, s=1.1, device="cpu"):
    """n draws of p(k) proportional to (k+1)^-s over [0, V) (rank = token id)."""
    k = torch.arange(V, dtype=torch.float64, device=device)
    p = (k + 1.0).pow(-s)
    p = (p / p.sum()).to(torch.float32)
    return torch.multinomial(p, n, replacement=True, generator=gen)


def make(name, device="cpu", scale=1.0, dtype=None, target_boost=40.0):
    """Build config `name` on `device`. Returns a dict with e [B,T,D], c [V,D], bias, targets [B,T]."""
    cfg = CONFIGS[name]
    idx = int(name[1:]) - 1
    gen = torch.Generator(device=device)
    gen.manual_seed(idx)
    B, T = cfg["B"], cfg["T"]
    if scale != 1.0:
        T = max(1, int(round(T * scale)))
    D, V = cfg["D"], cfg["V"]
    dt = dtype or cfg["dtype"]
    N = B * T
    f32 = dict(dtype=torch.float32, device=device)

    c = torch.randn((V, D), generator=gen, **f32).mul_(cfg["c_std"]).to(dt)
    if cfg["targets"] == "zipf":
        t = zipf_targets(gen, N, V, device=device)
    else:
        t = torch.randint(0, V, (N,), generator=gen, device=device)
    if cfg["peaked"]:
        cf = c.float()
        ct = cf[t]
        z = torch.randn((N, D), generator=gen, **f32)
        e = (0.5 * z + target_boost * ct / ct.pow(2).sum(dim=1, keepdim=True)).to(dt)
        del cf, ct, z
    else:
        e = torch.randn((N, D), generator=gen, **f32).to(dt)
    bias = None
    if cfg["bias_std"] is not None:
        bias = torch.randn((V,), generator=gen, **f32).mul_(cfg["bias_std"]).to(dt)

    t = t.to(torch.int64)
    if cfg.get("pad_tail"):
        tail = int(round(cfg["pad_tail"] * T / cfg["T"]))
        t = t.view(B, T)
        if tail > 0:
            t[:, T - tail:] = IGNORE
        t = t.reshape(-1)
    elif cfg["ignore_frac"] > 0:
        k = cfg["ignore_count"] if scale == 1.0 else max(1, int(round(cfg["ignore_frac"] * N)))
        pos = torch.randperm(N, generator=gen, device=device)[:k]
        t[pos] = IGNORE

    return dict(name=name, e=e.view(B, T, D), c=c, bias=bias, targets=t.view(B, T), N=N, D=D, V=V,
                reduction=cfg["reduction"], ignore_index=IGNORE, dtype=dt, description=NAMES[name])


def flops(N, D, V, skip=0.0, want_dc=True):
    """Algorithmic MFMA work of one fwd+bwd: 2NDV forward + 6NDV(1 - skip) backward
    (recompute, dE and dC; 4NDV(1 - skip) without dC)."""
    return 2.0 * N * D * V + (6.0 if want_dc else 4.0) * N * D * V * (1.0 - skip)


def min_bytes(N, D, V, esize=2, bias=False):
    """Minimum HBM traffic of one fwd+bwd: read E and C twice, write dE, dC (and dBias)."""
    b = 2 * (N * D + V * D) * esize + (N * D + V * D) * esize
    if bias:
        b += 3 * V * esize
    return float(b)


def describe(w):
    return f"{w['name']}: {w['description']}"


if __name__ == "__main__":
    for n in CONFIGS:
        w = make(n, scale=1 / 64 if n != "c1" else 1.0)
        print(describe(w), tuple(w["e"].shape), tuple(w["c"].shape), int((w["targets"] == IGNORE).sum()))
