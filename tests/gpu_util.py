"""Helpers shared by the GPU parity tests: bf16 bit views between torch and
numpy, and the synthetic inputs of the benchmark configurations (torch CPU
generator, then moved to the device)."""

import numpy as np
import torch


def bits(t):
    """A bf16 torch tensor (any device) as numpy uint16 bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(b, device):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)


def npy(t):
    return t.detach().contiguous().cpu().numpy()


def activation(m, k, seed=0, n_out=None, mult=30.0, scale=1.0):
    """x = randn(m, k) * scale with ``n_out`` outlier channels (default 1% of k)
    multiplied by ``mult``, rounded to bf16 (the benchmark recipe)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * scale
    n_out = max(1, round(0.01 * k)) if n_out is None else n_out
    if n_out:
        cols = torch.randperm(k, generator=g)[:n_out]
        x[:, cols] *= mult
    return x.to(torch.bfloat16)


def weight(n, k, seed=1, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, k, generator=g) * std).to(torch.bfloat16)


def mismatch(a, b):
    a, b = np.asarray(a), np.asarray(b)
    bad = np.argwhere(a != b)
    return f"{len(bad)} of {a.size} differ; first {bad[:5].tolist()}: " \
           f"{a[tuple(bad[:5].T)] if len(bad) else ''} vs {b[tuple(bad[:5].T)] if len(bad) else ''}"
