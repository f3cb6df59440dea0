"""CPU baseline for bench.py — TEST/MEASUREMENT INFRASTRUCTURE, NOT THE PRODUCT.

A float32 torch-CPU restatement of the reference's CPU path,
reference/_reference.py:5-48: materialise logits = e c^T (+ bias) (:24-26),
per-sample cross entropy (:28), ignore mask (:33-34), reduction (:36-44), and
autograd for dE / dC / dBias (the reference's tests take gradients the same way,
tests/test_gradients.py:38-44).  It is timed on the host's cores on a bounded
slice of a workload's tokens and reported as tokens/s; it is a baseline for
context only.
"""

import os
import time

import torch
import torch.nn.functional as F


def loss_and_grads(e, c, targets, bias=None, reduction="mean", ignore_index=-100):
    """One fwd+bwd on CPU in float32. Returns (loss, dE, dC, dBias)."""
    e = e.detach().float().requires_grad_(True)
    c = c.detach().float().requires_grad_(True)
    b = bias.detach().float().requires_grad_(True) if bias is not None else None
    logits = e @ c.T
    if b is not None:
        logits = logits + b[None, :]
    t = targets.reshape(-1)
    per = F.cross_entropy(logits, t.clamp(min=0), reduction="none")
    valid = (t != ignore_index) if ignore_index is not None else torch.ones_like(t, dtype=torch.bool)
    per = per * valid
    if reduction == "none":
        loss = per
        loss.backward(torch.ones_like(loss))
    elif reduction == "sum":
        loss = per.sum()
        loss.backward()
    else:
        loss = per.sum() / valid.sum().clamp(min=1)
        loss.backward()
    return loss.detach(), e.grad, c.grad, (b.grad if b is not None else None)


def time_tokens_per_s(e, c, targets, bias=None, reduction="mean", ignore_index=-100, rows=None,
                      budget_s=20.0, threads=None):
    """Time fwd+bwd of the first `rows` tokens on CPU; returns a result dict.

    The full vocabulary and hidden size are kept, so per-token cost matches the
    workload; only the number of tokens is bounded.
    """
    if not threads:
        # The CPUs this process may run on, capped by OMP_NUM_THREADS when the host sets it
        # (a GPU box shares its host's cores; os.cpu_count() reports all of them).
        threads = len(os.sched_getaffinity(0)) or 1
        omp = os.environ.get("OMP_NUM_THREADS", "")
        if omp.isdigit() and int(omp) > 0:
            threads = min(threads, int(omp))
    torch.set_num_threads(threads)
    e = e.reshape(-1, e.shape[-1])
    t = targets.reshape(-1)
    n = e.shape[0] if rows is None else min(rows, e.shape[0])
    e_s, t_s = e[:n].float().cpu(), t[:n].cpu()
    c_s = c.float().cpu()
    b_s = bias.float().cpu() if bias is not None else None
    loss_and_grads(e_s[: min(n, 8)], c_s, t_s[: min(n, 8)], b_s, reduction, ignore_index)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        loss_and_grads(e_s, c_s, t_s, b_s, reduction, ignore_index)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return dict(value=n * reps / el, unit="tokens/s", cores=threads, rows=n, reps=reps, seconds=el)
