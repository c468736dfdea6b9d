"""The packed weight (``pack_weight``; ``xpuint8_pack_weight_stream``): its
bytes against a torch restatement of the MFMA block layout, and every GEMM
that reads it -- the persistent kernel (config 3's shape and a ragged batch),
the split-K kernel (the N = 1280 shapes, a ragged one), both projections of
the FFN -- bit for bit the row-major weight's result and the oracle's; shapes
whose GEMMs read the weight row-major (K slices, the skinny kernel) through
the packed entry point; and the rules that decide when the copy is used (an
in-place write, an alias, an offset view, a module's weight moved or written,
a storage that is freed)."""

import gc

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import activation, bits, mismatch, npy, weight
from xpu_kernels import int8
from xpu_kernels.int8 import _lib as L
from xpu_kernels.int8 import ops

pytestmark = pytest.mark.gpu


def block_layout(w8):
    """w8 int8 [N, K] (N % 16 == 0, K % 16 == 0) in the MFMA block layout:
    16-row x 64-byte blocks, block (n/16, k/64) at ((n/16) * ceil(K/64) +
    k/64) * 1024, row r at 64r and at position p the row's 16-byte chunk
    p ^ ((r >> 1) & 3); zeros past K."""
    w = w8.cpu()
    n, k = w.shape
    kp = (k + 63) // 64 * 64
    if kp != k:
        w = torch.cat([w, torch.zeros(n, kp - k, dtype=torch.int8)], dim=1)
    b = w.reshape(n // 16, 16, kp // 64, 4, 16).permute(0, 2, 1, 3, 4)   # nb, kb, r, c, byte
    r = torch.arange(16).view(16, 1)
    p = torch.arange(4).view(1, 4)
    src = (p ^ ((r >> 1) & 3)).view(1, 1, 16, 4, 1).expand(n // 16, kp // 64, 16, 4, 16)
    return torch.gather(b, 3, src).reshape(-1)


@pytest.mark.parametrize("n,k", [(10240, 1280), (1280, 5120), (48, 1296), (16, 16), (32, 272)])
def test_pack_layout_exact(dev, n, k):
    g = torch.Generator().manual_seed(n + k)
    w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    lib = L._lib()
    need = lib.xpuint8_packed_weight_bytes(n, k)
    assert need == (n // 16) * ((k + 63) // 64) * 1024
    packed = torch.full((need,), 99, device=dev, dtype=torch.int8)
    wd = w8.to(dev)
    assert lib.xpuint8_pack_weight_stream(L._stream(dev), L._ptr(wd), L._ptr(packed), n, k) == 0, \
        lib.xpuint8_last_error()
    assert torch.equal(packed.cpu(), block_layout(w8))


def test_pack_rejects_bad_shapes(dev):
    lib = L._lib()
    assert lib.xpuint8_packed_weight_bytes(24, 64) == -1
    assert lib.xpuint8_packed_weight_bytes(16, 40) == -1
    w = torch.zeros(32, 64, device=dev, dtype=torch.int8)
    assert lib.xpuint8_pack_weight_stream(L._stream(dev), L._ptr(w), L._ptr(w), 24, 64) != 0
    assert b"multiples of 16" in lib.xpuint8_last_error()


def _both(dev, n, k, seed):
    """The same weight prepared with and without its packed copy."""
    w = weight(n, k, seed=seed).to(dev)
    w8p, ws = int8.prepare_weight(w)
    w8r, ws_r = int8.prepare_weight(w, pack=False)
    assert torch.equal(w8p, w8r) and torch.equal(ws, ws_r)
    assert ops._packed_for(w8p) is not None and ops._packed_for(w8r) is None
    return w8p, w8r, ws


# (M, N, K): the persistent kernel (config 3; a batch that is not a multiple
# of 256), the split-K kernel (the SDXL N = 1280 shapes; ragged rows and a
# last column tile of 16), K slices (M = 200, 512; M = 48 at N < 2048) and the
# skinny kernel reading the packed weight (M = 1, 7, 16, 48 at N >= 2048, 64;
# the row counts one m-block to four, N = 1296 a last weight block alone)
LINEAR_SHAPES = [(4096, 10240, 1280), (3000, 10240, 1280), (4096, 1280, 5120),
                 (4096, 1280, 2048), (4096, 1280, 1280), (2100, 1296, 2048), (200, 1280, 4096),
                 (512, 4096, 4096), (16, 4096, 4096), (1, 4096, 4096), (7, 1296, 2048),
                 (48, 2064, 1280), (64, 10240, 1280), (48, 1280, 5120)]


@pytest.mark.parametrize("m,n,k", LINEAR_SHAPES)
def test_linear_packed_equals_rowmajor(dev, m, n, k):
    w8p, w8r, ws = _both(dev, n, k, seed=n + 11)
    x = activation(m, k, seed=m + k).to(dev)
    bias = weight(1, n, seed=5, std=0.01)[0].to(dev)
    yp = int8.linear(x, w8p, ws, bias)
    yr = int8.linear(x, w8r, ws, bias)
    assert np.array_equal(bits(yp), bits(yr)), mismatch(bits(yp), bits(yr))


@pytest.mark.parametrize("m,n,k", [(4096, 10240, 1280), (4096, 1280, 1280), (1100, 1296, 2048),
                                   (16, 4096, 4096), (5, 1296, 1280)])
def test_linear_packed_exact(dev, m, n, k):
    w8p, _, ws = _both(dev, n, k, seed=n + 13)
    x = activation(m, k, seed=2 * m + k)
    bias = weight(1, n, seed=6, std=0.01)[0]
    y = int8.linear(x.to(dev), w8p, ws, bias.to(dev))
    want = O.linear(bits(x), npy(w8p), npy(ws), O.bf16_to_f32(bits(bias)))
    assert np.array_equal(bits(y), want), mismatch(bits(y), want)


def test_linear_gemm_packed_entry(dev):
    """xpuint8_linear_gemm_packed_stream against xpuint8_linear_gemm_tiled_stream
    (the block-layout x, row-major weight) at config 3 and a split-K shape, and
    against xpuint8_linear_gemm_stream at two skinny shapes."""
    lib = L._lib()
    for m, n, k in [(4096, 10240, 1280), (4096, 1280, 5120)]:
        w8p, _, ws = _both(dev, n, k, seed=n + 17)
        x = activation(m, k, seed=m + 3).to(dev)
        tb = ((m + 15) // 16) * ((k + 63) // 64) * 1024
        xq = torch.empty(tb, device=dev, dtype=torch.int8)
        xs = torch.empty(m, device=dev, dtype=torch.float32)
        st = L._stream(dev)
        assert lib.xpuint8_convrot_quantize_tiled_stream(st, L._ptr(x), L._ptr(xq), L._ptr(xs),
                                                         m, k) == 0
        b = weight(1, n, seed=8, std=0.01)[0].to(dev)
        o1 = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        o2 = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        assert lib.xpuint8_linear_gemm_tiled_stream(st, L._ptr(xq), L._ptr(xs), L._ptr(w8p),
                                                    L._ptr(ws), L._ptr(b), 1, L._ptr(o1),
                                                    m, n, k) == 0
        packed = ops._packed_for(w8p)
        assert lib.xpuint8_linear_gemm_packed_stream(st, L._ptr(xq), L._ptr(xs), L._ptr(packed),
                                                     L._ptr(ws), L._ptr(b), 1, L._ptr(o2),
                                                     m, n, k) == 0, lib.xpuint8_last_error()
        assert np.array_equal(bits(o1), bits(o2)), mismatch(bits(o1), bits(o2))
    # the skinny kernel (M = 16, 40) against xpuint8_linear_gemm_stream (q and
    # the weight row-major)
    for m, n, k in [(16, 4096, 4096), (40, 2064, 1280)]:
        w8p, _, ws = _both(dev, n, k, seed=n + 19)
        x = activation(m, k, seed=m + 5).to(dev)
        q, xs = int8.quantize(x)
        tb = ((m + 15) // 16) * ((k + 63) // 64) * 1024
        xq = torch.empty(tb, device=dev, dtype=torch.int8)
        xs_t = torch.empty(m, device=dev, dtype=torch.float32)
        st = L._stream(dev)
        assert lib.xpuint8_convrot_quantize_tiled_stream(st, L._ptr(x), L._ptr(xq),
                                                         L._ptr(xs_t), m, k) == 0
        assert torch.equal(xs, xs_t)
        b = weight(1, n, seed=8, std=0.01)[0].to(dev)
        o1 = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        o2 = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        assert lib.xpuint8_linear_gemm_stream(st, L._ptr(q), L._ptr(xs), L._ptr(w8p), L._ptr(ws),
                                              L._ptr(b), 1, L._ptr(o1), m, n, k) == 0
        assert lib.xpuint8_linear_gemm_packed_stream(
            st, L._ptr(xq), L._ptr(xs_t), L._ptr(ops._packed_for(w8p)), L._ptr(ws), L._ptr(b), 1,
            L._ptr(o2), m, n, k) == 0, lib.xpuint8_last_error()
        assert np.array_equal(bits(o1), bits(o2)), mismatch(bits(o1), bits(o2))
    # a shape whose GEMM reads neither block layout (K slices) is refused
    xq = torch.zeros(48 * 5120, device=dev, dtype=torch.int8)
    xs = torch.ones(48, device=dev)
    o = torch.empty((48, 1280), device=dev, dtype=torch.bfloat16)
    w8p, _, ws = _both(dev, 1280, 5120, seed=1)
    assert lib.xpuint8_linear_gemm_packed_stream(L._stream(dev), L._ptr(xq), L._ptr(xs),
                                                 L._ptr(ops._packed_for(w8p)), L._ptr(ws), None,
                                                 0, L._ptr(o), 48, 1280, 5120) != 0


# (M, K, inner, act): config 4 (GEGLU), a ragged batch, GELU-erf (an
# unpaired up-projection), and the skinny up-projection reading the packed
# weight: situ at 256 rows (two 128-row chunks) and K slices in the
# down-projection, GEGLU at one row and 129 (a chunk of one row), GELU-erf at
# 40 rows (unpaired)
@pytest.mark.parametrize("m,k,inner,act", [(4096, 1280, 5120, "geglu_erf"),
                                           (2100, 1280, 5120, "geglu_erf"),
                                           (4096, 1280, 5120, "gelu_erf"),
                                           (256, 1280, 5120, "situ"),
                                           (1, 1280, 5120, "geglu_erf"),
                                           (129, 1280, 5120, "geglu_erf"),
                                           (40, 1280, 5120, "gelu_erf")])
def test_ffn_packed_equals_rowmajor(dev, m, k, inner, act):
    up_rows = 2 * inner if act in ("geglu_erf", "situ") else inner
    up_p, up_r, us = _both(dev, up_rows, k, seed=up_rows + 1)
    dn_p, dn_r, ds = _both(dev, k, inner, seed=inner + 2)
    x = activation(m, k, seed=m + 7).to(dev)
    b = weight(1, k, seed=9, std=0.01)[0].to(dev)
    yp = int8.ffn(x, up_p, us, dn_p, ds, b, act=act)
    yr = int8.ffn(x, up_r, us, dn_r, ds, b, act=act)
    assert np.array_equal(bits(yp), bits(yr)), mismatch(bits(yp), bits(yr))
    # one weight packed, the other not
    ym = int8.ffn(x, up_r, us, dn_p, ds, b, act=act)
    assert np.array_equal(bits(ym), bits(yr)), mismatch(bits(ym), bits(yr))


def test_packed_copy_follows_inplace_writes(dev):
    n, k, m = 10240, 1280, 4096
    w8, ws = int8.prepare_weight(weight(n, k, seed=21).to(dev))
    x = activation(m, k, seed=22).to(dev)
    w8[100:116, :64] = 5                        # in place: the copy is stale from here
    assert ops._packed_for(w8) is None
    y_stale_safe = int8.linear(x, w8, ws)       # reads w8 itself
    w8r = w8.clone()
    y_ref = int8.linear(x, w8r, ws)
    assert np.array_equal(bits(y_stale_safe), bits(y_ref))
    assert int8.pack_weight(w8) and ops._packed_for(w8) is not None
    y_new = int8.linear(x, w8, ws)
    assert np.array_equal(bits(y_new), bits(y_ref)), mismatch(bits(y_new), bits(y_ref))


def test_packed_copy_aliases_and_views(dev):
    n, k = 4096, 1280
    w8, ws = int8.prepare_weight(weight(2 * n, k, seed=23).to(dev))
    assert ops._packed_for(w8.detach()) is not None         # an alias finds it
    assert ops._packed_for(w8[n:]) is None                  # offset view: not the packed rows
    assert ops._packed_for(w8[:n]) is None                  # another shape over the storage
    x = activation(4096, k, seed=24).to(dev)
    y = int8.linear(x, w8[n:], ws[n:])
    y_ref = int8.linear(x, w8[n:].clone(), ws[n:])
    assert np.array_equal(bits(y), bits(y_ref))
    key = w8.untyped_storage().data_ptr()
    assert key in ops._PACKED
    del w8, y
    gc.collect()
    assert key not in ops._PACKED                            # freed with the storage


def test_int8linear_packs_its_weight(dev):
    n, k = 10240, 1280
    w = weight(n, k, seed=25).to(dev)
    w8r, ws = int8.prepare_weight(w, pack=False)
    mod = int8.Int8Linear(w8r, ws, weight(1, n, seed=26, std=0.01)[0].to(dev))
    x = activation(4096, k, seed=27).to(dev)
    y1 = mod(x)                                              # packs on first use
    assert ops._packed_for(mod.w8) is not None
    y0 = int8.linear(x, w8r.clone(), ws, mod.bias)
    assert np.array_equal(bits(y1), bits(y0))
    with torch.no_grad():
        mod.w8[0, :16] = -3                                  # in place: packed again on use
    y2 = mod(x)
    y2_ref = int8.linear(x, mod.w8.clone(), ws, mod.bias)
    assert np.array_equal(bits(y2), bits(y2_ref))
    off = int8.Int8Linear(w8r.clone(), ws, pack=False)
    off(x)
    assert ops._packed_for(off.w8) is None


def nn_layout(w8):
    """w8 int8 [R, C] (C % 32 == 0) in the NN stage order of the split-K
    GEMM: per 64-row step s, 32-column group c and 32-row half h the 1 KB
    block ((s * C/32 + c) * 2 + h) * 1024, its 16-byte chunk l holding row l/2
    of the half and column half (l & 1) ^ ((l >> 5) & 1) of the group; zeros
    past R."""
    w = w8.cpu().numpy()
    r, c = w.shape
    rp = (r + 63) // 64 * 64
    wp = np.zeros((rp, c), np.int8)
    wp[:r] = w
    # [s, h, row in half, c group, column half, 16 bytes]
    v = wp.reshape(rp // 64, 2, 32, c // 32, 2, 16)
    l = np.arange(64)
    row, half = l >> 1, (l & 1) ^ ((l >> 5) & 1)
    blocks = v[:, :, row, :, half, :]                 # [l, s, h, cg, 16] (advanced index first)
    return torch.from_numpy(np.ascontiguousarray(blocks.transpose(1, 3, 2, 0, 4)).reshape(-1))


@pytest.mark.parametrize("r,c", [(5120, 1280), (2064, 1280), (48, 64)])
def test_pack_nn_layout_exact(dev, r, c):
    g = torch.Generator().manual_seed(r * 3 + c)
    w8 = torch.randint(-127, 128, (r, c), generator=g, dtype=torch.int8)
    lib = L._lib()
    need = lib.xpuint8_packed_weight_nn_bytes(r, c)
    assert need == (r + 63) // 64 * 64 * c
    packed = torch.full((need,), 99, device=dev, dtype=torch.int8)
    wd = w8.to(dev)
    assert lib.xpuint8_pack_weight_nn_stream(L._stream(dev), L._ptr(wd), L._ptr(packed), r, c) \
        == 0, lib.xpuint8_last_error()
    assert torch.equal(packed.cpu(), nn_layout(w8))
    assert lib.xpuint8_packed_weight_nn_bytes(64, 48) == -1


# (M, N, K) of dx = dy [M, N] against w8 [N, K]: config 5, a ragged batch, a
# contraction whose last 64-row step is partly past N (2064 = 32 * 64 + 16),
# and a batch small enough for the K-slice kernels (the packed form unused)
@pytest.mark.parametrize("m,n,k", [(4096, 5120, 1280), (3000, 5120, 1280), (4096, 2064, 1280),
                                   (256, 5120, 1280)])
def test_dx_int8_packed_equals_rowmajor(dev, m, n, k):
    w8p, w8r, ws = _both(dev, n, k, seed=n + 31)
    g = torch.Generator().manual_seed(m + n)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16).to(dev)
    dp = int8.linear_dx_int8(dy, w8p, ws)
    dr = int8.linear_dx_int8(dy, w8r, ws)
    assert np.array_equal(bits(dp), bits(dr)), mismatch(bits(dp), bits(dr))
    if m >= 4096 and n == 5120:
        assert ops._packed_entry(w8p)[4] is not None       # the NN form was made and used


def test_dx_int8_packed_exact(dev):
    m, n, k = 1536, 2064, 1280
    w8p, _, ws = _both(dev, n, k, seed=41)
    g = torch.Generator().manual_seed(42)
    dy = (torch.randn(m, n, generator=g) * 1e-3).to(torch.bfloat16)
    d = int8.linear_dx_int8(dy.to(dev), w8p, ws)
    want = O.linear_dx_int8(bits(dy), npy(w8p), npy(ws))
    assert np.array_equal(bits(d), want), mismatch(bits(d), want)


def test_int8_linear_backward_packed(dev):
    """The training step through autograd (int8 backward) with and without the
    packed forms: forward output and dx bit for bit."""
    m, n, k = 4096, 5120, 1280
    w8p, w8r, ws = _both(dev, n, k, seed=43)
    b = weight(1, n, seed=44, std=0.01)[0].to(dev)
    x = activation(m, k, seed=45).to(dev)
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(46)) * 1e-3) \
        .to(torch.bfloat16).to(dev)
    grads = []
    for w8 in (w8p, w8r):
        xx = x.clone().requires_grad_(True)
        y = int8.int8_linear(xx, w8, ws, b, mode="int8")
        y.backward(dy)
        grads.append((bits(y), bits(xx.grad)))
    assert np.array_equal(grads[0][0], grads[1][0])
    assert np.array_equal(grads[0][1], grads[1][1]), mismatch(grads[0][1], grads[1][1])


# linear with the residual update and linear_acc, each one library call that
# quantizes into the layout its GEMM reads: the persistent kernel (config 3;
# a ragged batch), the split-K kernel, and a batch whose GEMM reads the
# activation row-major (K slices)
ONE_CALL_SHAPES = [(4096, 10240, 1280), (3000, 10240, 1280), (4096, 1280, 5120), (200, 1280, 4096)]


@pytest.mark.parametrize("m,n,k", ONE_CALL_SHAPES)
def test_linear_residual_one_call(dev, m, n, k):
    w8p, w8r, ws = _both(dev, n, k, seed=n + 51)
    x = activation(m, k, seed=m + 52)
    bias = weight(1, n, seed=53, std=0.01)[0]
    g = torch.Generator().manual_seed(m + n)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    rscale = (torch.rand(n, generator=g) * 2 - 0.5).to(torch.bfloat16)
    args = dict(residual=res.to(dev), residual_scale=rscale.to(dev))
    yp = int8.linear(x.to(dev), w8p, ws, bias.to(dev), **args)
    yr = int8.linear(x.to(dev), w8r, ws, bias.to(dev), **args)
    assert np.array_equal(bits(yp), bits(yr)), mismatch(bits(yp), bits(yr))
    if m * n <= 4096 * 10240 and k <= 1280:
        d = O.linear(bits(x), npy(w8p), npy(ws), O.bf16_to_f32(bits(bias)))
        f = O.bf16_to_f32
        want = O.f32_to_bf16(f(bits(res)) + f(d) * f(bits(rscale))[None, :])
        assert np.array_equal(bits(yp), want), mismatch(bits(yp), want)


@pytest.mark.parametrize("m,n,k", ONE_CALL_SHAPES)
def test_linear_acc_one_call(dev, m, n, k):
    w8p, w8r, ws = _both(dev, n, k, seed=n + 61)
    x = activation(m, k, seed=m + 62)
    accp, xsp = int8.linear_acc(x.to(dev), w8p, ws)
    accr, xsr = int8.linear_acc(x.to(dev), w8r, ws)
    assert torch.equal(accp, accr) and torch.equal(xsp, xsr)
    acc2, xs2, ws2 = int8.linear(x.to(dev), w8p, ws, return_acc=True)
    assert torch.equal(acc2, accp) and torch.equal(xs2, xsp) and torch.equal(ws2, ws)
    q, s = O.convrot_quantize(bits(x))
    assert np.array_equal(npy(xsp), s)
    if k <= 1280:
        assert np.array_equal(npy(accp), O.int_mm(q, npy(w8p)))


@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16, torch.float16, None])
@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("mode,m", [("int8", 4096), ("dense", 4096), ("dense", 100)])
def test_backward_one_call(dev, bias_dtype, packed, mode, m):
    """The backward of int8_linear (dx and the bias gradient in one library
    call) against linear_dx_int8 -- or linear_dx of dequant_weight -- and
    column_sum called separately, bit for bit; the bias gradient in the
    bias's dtype, as autograd's cast of the bf16 sum gives it.  M = 100 splits
    the dense product's contraction across blocks."""
    n, k = 5120, 1280
    w8p, w8r, ws = _both(dev, n, k, seed=71)
    w8 = w8p if packed else w8r
    x = activation(m, k, seed=72).to(dev).requires_grad_(True)
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(73)) * 1e-3) \
        .to(torch.bfloat16).to(dev)
    bias = None
    if bias_dtype is not None:
        bias = (weight(1, n, seed=74, std=0.01)[0]).to(dev, bias_dtype).requires_grad_(True)
    y = int8.int8_linear(x, w8, ws, bias, mode=mode)
    y.backward(dy)
    if mode == "int8":
        dx_ref = int8.linear_dx_int8(dy, w8r, ws)
    else:
        dx_ref = int8.linear_dx(dy, int8.dequant_weight(w8r, ws))
    assert np.array_equal(bits(x.grad), bits(dx_ref)), mismatch(bits(x.grad), bits(dx_ref))
    if bias is not None:
        db_ref = ops.column_sum(dy).to(bias_dtype)
        assert bias.grad.dtype == bias_dtype
        assert torch.equal(bias.grad.view(torch.int32 if bias_dtype == torch.float32 else
                                          torch.int16),
                           db_ref.view(torch.int32 if bias_dtype == torch.float32 else
                                       torch.int16))
