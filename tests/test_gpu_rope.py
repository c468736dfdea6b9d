"""GPU parity of the RMSNorm + rope accumulator consumer against the oracle.

The reference checks its own kernel against its torch chain with a tolerance
(python/xpu_kernels/triton/reference.py:43-51, SAME_ARITHMETIC_REL = 1e-3 on
the relative norm of the difference): the row sum's order and the rsqrt are
implementation choices.  The same bar here, plus: every head row within 2^-6 of
its largest output, and at least 95% of the outputs bit-identical."""

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import bits, npy
from xpu_kernels import rope

SAME_ARITHMETIC_REL = 1e-3


def _freqs(rng, fb, fs, d):
    theta = rng.uniform(-np.pi, np.pi, (fb, fs, 1, d // 2))
    c, s = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    return np.stack([np.stack([c, -s], -1), np.stack([s, c], -1)], -2)


def _check(got, want):
    g = O.bf16_to_f32(got).astype(np.float64)
    w = want.astype(np.float64)
    rel = np.linalg.norm(g - w) / np.linalg.norm(w)
    assert rel <= SAME_ARITHMETIC_REL, rel
    row_max = np.abs(w).max(-1, keepdims=True)
    assert np.all(np.abs(g - w) <= 2.0 ** -6 * row_max), np.max(np.abs(g - w) / row_max)
    same = np.mean(O.f32_to_bf16(want) == got)
    assert same >= 0.95, same


CASES = [
    # B, S, H, D, split_half, freqs batch, freqs seq, accumulator columns (qkv width)
    (1, 512, 24, 128, True, 1, 512, 3 * 24 * 128),
    (2, 64, 3, 256, False, 2, 64, 3 * 256),
    (3, 5, 1, 2, True, 1, 1, 2),
    (2, 33, 7, 96, True, 2, 1, 7 * 96 + 16),
    # the 16-byte vector kernel (D = 64 or 128): interleaved pairs, a partial
    # last wave of heads, broadcast rotations, a padded accumulator row
    (2, 64, 5, 128, False, 1, 64, 5 * 128),
    (1, 128, 24, 64, True, 1, 1, 3 * 24 * 64),
    (2, 40, 9, 64, False, 2, 40, 9 * 64 + 64),
    (1, 16, 64, 128, True, 1, 16, 64 * 128),
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,H,D,split,fb,fs,width", CASES)
def test_rms_rope_dequant_matches_oracle(dev, B, S, H, D, split, fb, fs, width):
    rng = np.random.default_rng(B * 1000 + S + H + D)
    full = rng.integers(-2 ** 17, 2 ** 17, (B, S, width)).astype(np.int32)
    xs = rng.uniform(0.005, 0.05, (B, S)).astype(np.float32)
    ws = rng.uniform(1e-5, 1e-4, H * D).astype(np.float32)
    scale = O.bf16_round(rng.uniform(0.5, 1.5, D).astype(np.float32))
    f = _freqs(rng, fb, fs, D)
    acc_full = torch.from_numpy(full).to(dev)
    acc = acc_full[..., : H * D].view(B, S, H, D) if width == H * D else \
        acc_full[..., : H * D].unflatten(-1, (H, D))
    out = rope.rows_dq(acc, torch.from_numpy(f).to(dev), torch.from_numpy(scale).to(dev), 1e-6,
                       torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev), split)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (B, S, H, D)
    want = O.rms_rope_dequant(full[..., : H * D].reshape(B, S, H, D), xs, ws, f, scale,
                              1e-6, split)
    _check(bits(out), want)


@pytest.mark.gpu
def test_q_and_k_from_one_qkv_accumulator(dev):
    """rms_rope_split_half_dequant on the q and k slices of a [B, S, 3*H*D]
    accumulator, with their own column and norm scales."""
    B, S, H, D = 2, 40, 4, 64
    rng = np.random.default_rng(7)
    full = rng.integers(-2 ** 16, 2 ** 16, (B, S, 3 * H * D)).astype(np.int32)
    xs = rng.uniform(0.01, 0.05, (B, S)).astype(np.float32)
    qw, kw = (rng.uniform(1e-5, 1e-4, H * D).astype(np.float32) for _ in range(2))
    qs, ks = (O.bf16_round(rng.uniform(0.5, 1.5, D).astype(np.float32)) for _ in range(2))
    f = _freqs(rng, 1, S, D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    acc = t(full)
    q_acc = acc[..., : H * D].unflatten(-1, (H, D))
    k_acc = acc[..., H * D: 2 * H * D].unflatten(-1, (H, D))
    q, k = rope.rms_rope_split_half_dequant(q_acc, k_acc, t(f), t(qw), t(kw), t(xs), t(qs),
                                            t(ks))
    _check(bits(q), O.rms_rope_dequant(full[..., : H * D].reshape(B, S, H, D), xs, qw, f, qs))
    _check(bits(k), O.rms_rope_dequant(full[..., H * D: 2 * H * D].reshape(B, S, H, D), xs, kw,
                                       f, ks))


@pytest.mark.gpu
def test_rope_argument_errors(dev):
    acc = torch.zeros((1, 4, 2, 8), dtype=torch.int32, device=dev)
    f = torch.zeros((1, 4, 1, 4, 2, 2), device=dev)
    ones = lambda n: torch.ones(n, device=dev)
    with pytest.raises(ValueError):
        rope.rows_dq(acc, f, ones(8), 1e-6, ones(4), ones(15))          # w_scale size
    with pytest.raises(ValueError):
        rope.rows_dq(acc, f[..., :3, :, :], ones(8), 1e-6, ones(4), ones(16))
    with pytest.raises(TypeError):
        rope.rows_dq(acc.float(), f, ones(8), 1e-6, ones(4), ones(16))
