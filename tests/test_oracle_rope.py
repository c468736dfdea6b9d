"""Pins of the oracle's RMSNorm + rope restatement (oracle/rope.py) by
closed forms -- not by retyping its formula:
* identity rotation and unit scale leave x / rms(x), checked in float64;
* a constant row normalizes to +-1;
* a pair (1, 1) rotated by theta is (cos - sin, sin + cos);
* the rotation keeps every pair's length;
* split-half and interleaved pairing agree under the dim permutation;
* the dequant step is the epilogue's expression (float64 within one rounding)."""

import numpy as np

import oracle as O

BF16_ULP = 2.0 ** -7       # relative spacing bound of bf16 values


def _bf16(x):
    return O.bf16_round(np.asarray(x, dtype=np.float32))


def _freqs(theta):
    """freqs_cis [1, 1, 1, P, 2, 2] of rotations by theta[p]."""
    c, s = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    f = np.stack([np.stack([c, -s], -1), np.stack([s, c], -1)], -2)
    return f[None, None, None]


def test_identity_rotation_is_the_rms_norm():
    rng = np.random.default_rng(0)
    B, S, H, D = 2, 3, 4, 64
    x = _bf16(rng.standard_normal((B, S, H, D)) * 3)
    out = O.rms_rope_bf16(x, _freqs(np.zeros(D // 2)), np.ones(D, np.float32), eps=1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 ** 2, -1, keepdims=True) + 1e-6)
    # two bf16 roundings (y, then the rotated value) plus fp32 noise
    assert np.all(np.abs(out - want) <= 2 * BF16_ULP * np.abs(want) + 1e-30)


def test_constant_row_normalizes_to_unit():
    D = 32
    for c in (3.0, -0.125, 1000.0):
        x = np.full((1, 1, 1, D), c, np.float32)
        out = O.rms_rope_bf16(x, _freqs(np.zeros(D // 2)), np.ones(D, np.float32))
        assert np.all(out == np.sign(c))


def test_rotating_a_unit_pair():
    D = 16
    theta = np.linspace(0.1, 3.0, D // 2)
    x = np.ones((1, 1, 1, D), np.float32)
    out = O.rms_rope_bf16(x, _freqs(theta), np.ones(D, np.float32))[0, 0, 0]
    c, s = np.cos(theta), np.sin(theta)
    for got, want in ((out[: D // 2], c - s), (out[D // 2:], s + c)):
        assert np.all(np.abs(got - want) <= BF16_ULP * np.abs(want) + 2 ** -20)


def test_rotation_keeps_pair_lengths():
    rng = np.random.default_rng(1)
    D = 128
    x = _bf16(rng.standard_normal((3, 5, 2, D)))
    f = _freqs(rng.uniform(-np.pi, np.pi, D // 2))
    scale = _bf16(rng.uniform(0.5, 1.5, D))
    y = O.rms_rope_bf16(x, _freqs(np.zeros(D // 2)), scale)
    o = O.rms_rope_bf16(x, f, scale)
    ny = np.hypot(y[..., : D // 2], y[..., D // 2:])
    no = np.hypot(o[..., : D // 2], o[..., D // 2:])
    assert np.all(np.abs(no - ny) <= 3 * BF16_ULP * ny + 1e-6)


def test_split_half_and_interleaved_agree():
    rng = np.random.default_rng(2)
    D = 64
    x = _bf16(rng.standard_normal((2, 2, 3, D)))
    f = _freqs(rng.uniform(-3, 3, D // 2))
    scale = _bf16(rng.uniform(0.5, 1.5, D))
    perm = np.empty(D, int)
    perm[0::2], perm[1::2] = np.arange(D // 2), np.arange(D // 2) + D // 2
    split = O.rms_rope_bf16(x, f, scale, split_half=True)
    inter = O.rms_rope_bf16(x[..., perm], f, scale[perm], split_half=False)
    assert np.array_equal(inter, split[..., perm])


def test_dequant_step():
    rng = np.random.default_rng(3)
    B, S, H, D = 2, 2, 2, 8
    acc = rng.integers(-2 ** 20, 2 ** 20, (B, S, H, D)).astype(np.int32)
    xs = rng.uniform(0.01, 0.1, (B, S)).astype(np.float32)
    ws = rng.uniform(1e-5, 1e-4, H * D).astype(np.float32)
    f = _freqs(np.zeros(D // 2))
    got = O.rms_rope_dequant(acc, xs, ws, f, np.ones(D, np.float32))
    x = acc.astype(np.float64) * (ws.reshape(H, D)[None, None] * xs[:, :, None, None])
    want = x / np.sqrt(np.mean(x ** 2, -1, keepdims=True) + 1e-6)
    assert np.all(np.abs(got - want) <= 3 * BF16_ULP * np.abs(want) + 1e-30)
