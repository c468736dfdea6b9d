"""Pins for the oracle's 256-point block Hadamard (oracle.hadamard256).

The oracle fixes the reference's fp32 operation order (src/xpuint8.cpp:75-83,
279-301, 441-448); these checks tie it to what the mathematics fixes, so that
a wrong digit mapping, sign, transposed factor or dropped term fails:

* the explicit matrix kron(H4,H4,H4,H4)/16 in float64 (docs/architecture.md:29-35);
* exact known answers: the all-ones vector is a fixed point, H e_j = +-1/16
  with the kron signs (so oracle(I) == H bit for bit);
* H is symmetric and involutory (ops.py:130-133: rotate(rotate(x)) == x) and
  orthogonal;
* a literal restatement of the reference's lane-per-group loops
  (``convrot_body``, src/xpuint8.cpp:325-336) on scalar registers.
"""

import numpy as np

import oracle as O


def test_explicit_matrix_matches():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((16, 1024)) * rng.uniform(0.01, 30, (16, 1))).astype(np.float32)
    got = O.hadamard256(x).astype(np.float64)
    h = O.hadamard256_matrix()
    want = (x.astype(np.float64).reshape(16, 4, 256) @ h.T).reshape(16, 1024)
    scale = np.abs(x).max(axis=1, keepdims=True)
    assert np.max(np.abs(got - want) / scale) < 4e-7


def test_matrix_is_kron_of_h4():
    h = O.hadamard256_matrix()
    i = np.arange(256)
    d = [(i >> (2 * k)) & 3 for k in range(4)]
    want = np.ones((256, 256))
    for k in range(4):
        want = want * O.H4[d[k][:, None], d[k][None, :]]
    assert np.array_equal(h, want / 16.0)


def test_all_ones_is_a_fixed_point_exactly():
    ones = np.ones((3, 512), dtype=np.float32)
    assert np.array_equal(O.hadamard256(ones), ones)
    # and so is a constant row of any (normal) magnitude
    c = np.full((1, 256), -3.75, dtype=np.float32)
    assert np.array_equal(O.hadamard256(c), c)


def test_unit_vectors_give_the_matrix_exactly():
    got = O.hadamard256(np.eye(256, dtype=np.float32)).astype(np.float64)
    h = O.hadamard256_matrix()
    assert np.array_equal(got, h.T)          # row j = H e_j
    assert np.array_equal(h, h.T)            # symmetric
    assert set(np.unique(np.abs(got))) == {1.0 / 16}


def test_involution_and_norm():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 768)).astype(np.float32)
    y = O.hadamard256(x)
    assert np.allclose(O.hadamard256(y), x, atol=2e-6, rtol=0)
    ng = np.linalg.norm(x.reshape(8, 3, 256), axis=-1)
    assert np.allclose(np.linalg.norm(y.reshape(8, 3, 256), axis=-1), ng, rtol=1e-6)


def test_groups_are_independent():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 1280)).astype(np.float32)
    y = O.hadamard256(x)
    for g in range(5):
        assert np.array_equal(y[:, 256 * g:256 * (g + 1)],
                              O.hadamard256(x[:, 256 * g:256 * (g + 1)]))


def _literal_group(v):
    """The reference's lane-per-group transform, loop for loop, in float32
    scalars: inreg on each of the 16 registers, then bfly4 over {b..b+3} and
    over {c, c+4, c+8, c+12} (src/xpuint8.cpp:78-83, 279-301, 328-336)."""
    f = np.float32
    H4 = [[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]]
    c = [[f(0.5 * H4[t & 3][k]) for t in range(16)] for k in range(4)]
    d = [[f(0.5 * H4[(t >> 2) & 3][k]) for t in range(16)] for k in range(4)]
    W = [[f(v[16 * w + q]) for q in range(16)] for w in range(16)]

    def inreg(r):
        t = [c[0][q] * r[(q & ~3) + 0] for q in range(16)]
        for k in range(1, 4):
            t = [t[q] + c[k][q] * r[(q & ~3) + k] for q in range(16)]
        u = [d[0][q] * t[(q & 3) + 0] for q in range(16)]
        for k in range(1, 4):
            u = [u[q] + d[k][q] * t[(q & 3) + 4 * k] for q in range(16)]
        return u

    def bfly4(a0, a1, a2, a3):
        h = f(0.5)
        out = [[None] * 16 for _ in range(4)]
        for q in range(16):
            p, m = a0[q] + a1[q], a0[q] - a1[q]
            qq, n = a2[q] + a3[q], a2[q] - a3[q]
            out[0][q], out[1][q] = (p + n) * h, (p - n) * h
            out[2][q], out[3][q] = (m + qq) * h, (qq - m) * h
        return out

    for b in range(0, 16, 4):
        for j in range(4):
            W[b + j] = inreg(W[b + j])
        W[b], W[b + 1], W[b + 2], W[b + 3] = bfly4(W[b], W[b + 1], W[b + 2], W[b + 3])
    for k in range(4):
        W[k], W[k + 4], W[k + 8], W[k + 12] = bfly4(W[k], W[k + 4], W[k + 8], W[k + 12])
    return np.array([W[w][q] for w in range(16) for q in range(16)], dtype=np.float32)


def test_literal_lane_per_group_loops_bit_for_bit():
    rng = np.random.default_rng(3)
    for s in (1.0, 1e-3, 250.0):
        v = (rng.standard_normal(256) * s).astype(np.float32)
        v = O.bf16_round(v)
        assert np.array_equal(_literal_group(v).view(np.uint32),
                              O.hadamard256(v[None, :])[0].view(np.uint32))


def test_operation_order_is_observable():
    """The bit-exact GPU comparison is meaningful only if a different (but
    mathematically equal) add order gives different bits on ordinary data."""
    rng = np.random.default_rng(4)
    x = O.bf16_round(rng.standard_normal((64, 256)).astype(np.float32) * 3)
    h = O.hadamard256_matrix().astype(np.float32)
    other = (x @ h.T).astype(np.float32)       # a BLAS order
    assert not np.array_equal(other.view(np.uint32), O.hadamard256(x).view(np.uint32))


# ------------------------------------------------ the kernels' two operation orders
def _unscaled(v):
    """The reference's operation order with every factor 0.5 dropped (the
    kernels' fast path): chains with coefficients +-1 on axes 0 and 1, the
    butterflies without their final halving on axes 2 and 3.  Its result is
    16 times the rotation wherever nothing overflows."""
    v = np.asarray(v, dtype=np.float32)
    k = v.shape[-1]
    r = v.reshape(-1, k // 256, 16, 4, 4)
    t = np.empty_like(r)
    for o in range(4):
        acc = O.H4[o, 0] * r[..., 0]
        for c in range(1, 4):
            acc = acc + O.H4[o, c] * r[..., c]
        t[..., o] = acc
    u = np.empty_like(t)
    for o in range(4):
        acc = O.H4[o, 0] * t[..., 0, :]
        for c in range(1, 4):
            acc = acc + O.H4[o, c] * t[..., c, :]
        u[..., o, :] = acc

    def bfly(a0, a1, a2, a3):
        p, m, q, n = a0 + a1, a0 - a1, a2 + a3, a2 - a3
        return p + n, p - n, m + q, q - m

    w = u.reshape(-1, k // 256, 4, 4, 16)
    w = np.stack(bfly(w[:, :, :, 0], w[:, :, :, 1], w[:, :, :, 2], w[:, :, :, 3]), axis=3)
    w = np.stack(bfly(w[:, :, 0], w[:, :, 1], w[:, :, 2], w[:, :, 3]), axis=2)
    return w.reshape(v.shape)


def _bf16_rows(rng, rows, lo_exp, hi_exp):
    """bf16 rows of random sign and mantissa whose exponents span [lo_exp, hi_exp)."""
    e = rng.integers(lo_exp, hi_exp, (rows, 256)).astype(np.float64)
    x = rng.choice([-1.0, 1.0], (rows, 256)) * rng.uniform(1, 2, (rows, 256)) * 2.0 ** e
    return O.bf16_round(x.astype(np.float32))


def test_unscaled_order_is_exact_below_two_to_120():
    """The fast path's claim: for every group with max|x| < 2^120 the unscaled
    order gives exactly 16 x the reference's result, across the whole bf16
    range below that bound, subnormal inputs included."""
    rng = np.random.default_rng(5)
    with np.errstate(over="ignore", invalid="ignore"):
        for lo, hi in ((-133, -126), (-140, -100), (-60, 60), (100, 119), (118, 120)):
            x = _bf16_rows(rng, 64, lo, hi)
            x[np.abs(x) >= 2.0 ** 120] = np.float32(2.0 ** 119)
            x[0] = np.float32(-(2.0 - 2.0 ** -7) * 2.0 ** 119)      # largest magnitude below the bound
            x[1] = O.bf16_round(np.full(256, 2.0 ** -133, np.float32))   # smallest bf16 subnormal
            ref = O.hadamard256(x)
            fast = _unscaled(x) * np.float32(0.0625)
            assert np.isfinite(fast).all()
            assert np.array_equal(fast.view(np.uint32), ref.view(np.uint32)), (lo, hi)


def test_unscaled_order_overflows_above_two_to_120():
    """Why the kernels keep the reference's scaled order for larger inputs: a
    constant row of 2^124 is a fixed point of the reference's chain, but its
    unscaled sums reach 2^128 = inf."""
    c = np.full((1, 256), 2.0 ** 124, np.float32)
    assert np.array_equal(O.hadamard256(c), c)
    with np.errstate(over="ignore"):
        assert np.isinf(_unscaled(c)).all()
