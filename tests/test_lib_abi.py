"""The C ABI without a GPU: the library loads, exports every function
include/xpuint8.h declares, and rejects bad arguments with the documented
codes and messages before touching a device (the reference's return-code
convention, src/xpuint8.cpp:733-776, 999-1002)."""

import ctypes
import os
import re

import pytest
import torch

from xpu_kernels.int8 import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "xpuint8.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(xpuint8_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    path = L.library_path()
    assert path is not None, "libxpuint8.so is not built (run __graft_entry__.build())"
    return L.open_library(path)


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = _declared()
    assert len(names) >= 25
    sigs = L._signatures()
    for n in names:
        assert hasattr(lib, n), n
        assert n in sigs, f"{n} has no ctypes signature in _lib.py"
    assert set(sigs) == set(names)


def test_group_size(lib):
    assert lib.xpuint8_convrot_groupsize() == 256


def test_c_consumer_is_built_and_links():
    """The plain C caller (tests/c_abi/linear_consumer.c) is built with the
    library and its dynamic links resolve: run without arguments it prints
    its usage before any HIP call."""
    import subprocess
    binp = os.path.join(ROOT, "tests", "c_abi", "linear_consumer")
    assert os.path.exists(binp), "not built (run __graft_entry__.build())"
    r = subprocess.run([binp], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr, r.stderr


P = ctypes.c_void_p(0x1000)   # never dereferenced: validation runs first
Z = ctypes.c_void_p(0)


def _rc(lib, fn, *args):
    rc = getattr(lib, fn)(*args)
    return rc, lib.xpuint8_last_error().decode()


@pytest.mark.parametrize("fn,args,code,substr", [
    ("xpuint8_convrot_quantize_stream", (Z, P, P, P, 4, 384), 3, "256"),
    ("xpuint8_convrot_quantize_stream", (Z, P, P, P, 0, 512), 2, "positive"),
    ("xpuint8_convrot_quantize_stream", (Z, Z, P, P, 4, 512), 6, "null"),
    ("xpuint8_convrot_quantize_act_stream", (Z, P, P, P, 4, 512, 9), 6, "activation"),
    ("xpuint8_convrot_rotate_bf16_stream", (Z, P, P, 4, 100), 3, "256"),
    ("xpuint8_dequant_epilogue_stream", (Z, P, P, P, P, Z, 4, 24), 2, "16"),
    ("xpuint8_dequant_epilogue_slice_stream", (Z, P, P, P, P, Z, 4, 32, 16), 2, "stride"),
    ("xpuint8_dequant_act_quantize_stream", (Z, P, P, P, P, P, 4, 512, 1), 6, "activation"),
    ("xpuint8_dequant_weight_stream", (Z, P, P, P, 0, 512), 2, "positive"),
    ("xpuint8_int8_gemm_stream", (Z, P, P, P, 4, 32, 24), 2, "16"),
    ("xpuint8_int8_gemm_stream", (Z, P, P, P, 4, 32, 1 << 20), 4, "131072"),
    ("xpuint8_int8_gemm_nn_stream", (Z, P, P, P, 4, 32, 32, Z), 6, "null"),
    ("xpuint8_linear_gemm_stream", (Z, P, P, P, P, Z, 0, P, 4, 24, 512), 2, "16"),
    ("xpuint8_linear_gemm_stream", (Z, P, P, P, P, Z, 2, P, 4, 32, 512), 2, "bias_bf16"),
    ("xpuint8_ffn_up_stream", (Z, P, P, P, P, P, 4, 512, 512, 2), 6, "activation"),
    ("xpuint8_ffn_up_stream", (Z, P, P, P, P, P, 4, 24, 512, 4), 2, "16"),
    ("xpuint8_ffn_up_stream", (Z, P, P, Z, P, P, 4, 512, 512, 4), 6, "null"),
    ("xpuint8_ffn_stream", (Z, P, P, P, P, P, Z, 0, P, 4, 512, 512, 2, P, 1 << 24), 6, "activation"),
    ("xpuint8_ffn_stream", (Z, P, P, P, P, P, Z, 0, P, 4, 400, 512, 4, P, 1 << 24), 3, "256"),
    ("xpuint8_ffn_stream", (Z, P, P, P, P, P, Z, 0, P, 4, 512, 300, 4, P, 1 << 24), 3, "256"),
    ("xpuint8_ffn_stream", (Z, P, P, P, Z, P, Z, 0, P, 4, 512, 512, 4, P, 1 << 24), 6, "null"),
    ("xpuint8_ffn_stream", (Z, P, P, P, P, P, Z, 2, P, 4, 512, 512, 4, P, 1 << 24), 2, "bias_bf16"),
    ("xpuint8_ffn_stream", (Z, P, P, P, P, P, Z, 0, P, 4, 512, 512, 4, P, 64), 2, "workspace_size"),
    ("xpuint8_dx_gemm_stream", (Z, P, P, P, P, 4, 24, 512, P), 2, "16"),
    ("xpuint8_linear_dx_int8_stream", (Z, P, P, P, P, 4, 32, 300, P, 1 << 20), 3, "256"),
    ("xpuint8_linear_dx_int8_stream", (Z, P, P, P, P, 4, 24, 512, P, 1 << 20), 2, "16"),
    ("xpuint8_linear_dx_int8_stream", (Z, P, P, P, P, 4, 32, 512, Z, 1 << 20), 6, "null"),
    ("xpuint8_linear_dx_int8_stream", (Z, P, P, P, P, 4, 32, 512, P, 1024), 2, "workspace_size"),
    ("xpuint8_linear_stream", (Z, P, P, P, Z, 0, P, 4, 32, 300, P, 1 << 20), 3, "256"),
    ("xpuint8_linear_stream", (Z, P, P, P, Z, 0, P, 4, 24, 512, P, 1 << 20), 2, "16"),
    ("xpuint8_linear_stream", (Z, P, P, P, Z, 2, P, 4, 32, 512, P, 1 << 20), 2, "bias_bf16"),
    ("xpuint8_linear_stream", (Z, P, P, P, Z, 0, P, 4, 32, 512, Z, 1 << 20), 6, "null"),
    ("xpuint8_linear_stream", (Z, P, P, P, Z, 0, P, 4, 32, 512, P, 64), 2, "workspace_size"),
    ("xpuint8_prepare_weight_stream", (Z, P, P, P, 16, 300), 3, "256"),
    ("xpuint8_quantize_row_stream", (Z, P, Z, P, P, 4, 20), 2, "16"),
    ("xpuint8_activation_table", (7 + 1, P), 6, "0..6"),
    ("xpuint8_linear_dw_stream", (Z, P, P, P, 64, 24, 32), 2, "16"),
    ("xpuint8_linear_dw_stream", (Z, P, Z, P, 64, 32, 32), 6, "null"),
])
def test_argument_errors_are_reported_without_a_device(lib, fn, args, code, substr):
    rc, msg = _rc(lib, fn, *args)
    assert rc == code and substr in msg, (rc, msg)


def test_errors_are_per_thread(lib):
    import threading
    rc, _ = _rc(lib, "xpuint8_convrot_quantize_stream", Z, P, P, P, 4, 384)
    seen = {}

    def other():
        lib.xpuint8_dequant_epilogue_stream(Z, P, P, P, P, Z, 4, 24)
        seen["msg"] = lib.xpuint8_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "16" in seen["msg"]
    assert "256" in lib.xpuint8_last_error().decode()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_init_without_a_device_fails_cleanly(lib):
    rc = lib.xpuint8_init()
    assert rc == 1 and "device" in lib.xpuint8_last_error().decode().lower()


def up256(b):
    return (b + 255) // 256 * 256


def tiled(m, k):
    """Bytes of an int8 [m, k] operand in the MFMA block layout: 16-row x
    64-byte blocks of 1 KB."""
    return -(-m // 16) * -(-k // 64) * 1024


def test_dx_workspace_size(lib):
    """The linear_dx_int8 workspace: q [M,N] int8 (row-major or in the block
    layout, whichever is larger), a [M] fp32, w8^T [K,N] int8 and the bf16
    [M,K] product, each rounded up to 256 bytes; -1 for a shape the entry
    point rejects."""
    m, n, k = 4096, 5120, 1280
    want = up256(m * n) + up256(4 * m) + up256(n * k) + up256(2 * m * k)
    assert lib.xpuint8_linear_dx_int8_workspace_size(m, n, k) == want
    assert lib.xpuint8_linear_dx_int8_workspace_size(3, 16, 256) == (
        up256(tiled(3, 16)) + 256 + 16 * 256 + up256(2 * 3 * 256))
    # a contraction split across blocks: then the slices' int32 [M,K] partials
    for m, n, k in [(1024, 5120, 1280), (200, 5120, 1280)]:
        s = k_slices(m, k, n)
        assert s in (4, 8)
        want = (up256(max(m * n, tiled(m, n))) + up256(4 * m) + up256(n * k) + up256(2 * m * k)
                + s * m * k * 4)
        assert lib.xpuint8_linear_dx_int8_workspace_size(m, n, k) == want, (m, n, k)
    assert lib.xpuint8_linear_dx_int8_workspace_size(4, 24, 512) == -1
    assert lib.xpuint8_linear_dx_int8_workspace_size(4, 32, 300) == -1


def k_slices(m, n, k):
    """The K slices of a product split across blocks.  First the skinny
    kernel's, for 33 <= m <= 128 (at m <= 64 only with n < 2048): the fewest
    power-of-two slices giving at least 256 blocks of 32 output columns, each
    slice a whole number of 64-byte steps and at least 1024 long.  Otherwise,
    when the 128 x 160 output tiles number below 128, the fewest power-of-two
    slices giving at least 192 blocks, each slice a whole number of 64-byte
    steps and at least 1024 long -- for m <= 256 counted in 128 x 128 tiles
    with slices down to 512 long; 0 when none applies (m <= 64 included)."""
    if k % 64:
        return 0
    if 32 < m <= 128 and (m > 64 or n < 2048):
        blocks, s = -(-n // 32), 1
        while blocks * s < 256 and (k // 64) % (2 * s) == 0 and k // (2 * s) >= 1024:
            s *= 2
        if s > 1:
            return s
    if m <= 64:
        return 0
    tiles = -(-m // 128) * -(-n // 160)
    if tiles >= 128:
        return 0
    least = 1024
    if m <= 256:
        tiles, least = -(-m // 128) * -(-n // 128), 512
    s = 1
    while tiles * s < 192 and (k // 64) % (2 * s) == 0 and k // (2 * s) >= least:
        s *= 2
    return s if s > 1 else 0


def test_linear_dx_workspace_size(lib):
    """The dense dx's optional workspace: fp32 [M, K] partial sums per slice
    when its 128 x 160 output tiles number below 128 (the fewest power-of-two
    slices giving 192 blocks, each a whole number of 32-row steps of at least
    1024 rows), else 0; -1 for a shape the entry point rejects."""
    assert lib.xpuint8_linear_dx_workspace_size(1024, 5120, 1280) == 4 * 1024 * 1280 * 4
    assert lib.xpuint8_linear_dx_workspace_size(200, 2048, 1280) == 2 * 200 * 1280 * 4
    assert lib.xpuint8_linear_dx_workspace_size(4096, 5120, 1280) == 0     # 256 tiles
    assert lib.xpuint8_linear_dx_workspace_size(64, 5120, 1280) == 0       # M <= 64
    assert lib.xpuint8_linear_dx_workspace_size(300, 1040, 272) == 0       # 1040 % 32
    assert lib.xpuint8_linear_dx_workspace_size(4, 24, 512) == -1
    # a slice's w rows past 2^32 bytes (2 slices of 107520 rows x 20000):
    # the unsplit kernel, no workspace
    assert lib.xpuint8_linear_dx_workspace_size(100, 215040, 20000) == 0


def test_linear_workspace_size(lib):
    """The linear's workspace: the quantized activation (row-major or in the
    block layout, whichever is larger) rounded up to 256 bytes, then its fp32
    row scales; for a product split in K across blocks, then (from a 256-byte
    boundary) the slices' int32 [M, N] partial products; -1 for a shape the
    entry point rejects."""
    shapes = [(4096, 1280, 5120), (4096, 10240, 1280), (3, 16, 256), (2100, 1296, 2304),
              (1024, 1280, 5120), (2048, 640, 5120), (1000, 1296, 4096), (1024, 1280, 1280),
              (128, 4096, 4096), (200, 160, 16384), (65, 4096, 1024), (64, 1280, 5120),
              (100, 1280, 5120), (48, 3072, 3072), (16, 1280, 5120), (128, 5120, 1280)]
    assert [k_slices(*s) for s in shapes] == [0, 0, 0, 0, 4, 4, 4, 0, 2, 32, 2, 4, 4, 0, 0, 2]
    for m, n, k in shapes:
        want = up256(max(m * k, tiled(m, k))) + 4 * m
        if k_slices(m, n, k):
            want = up256(want) + k_slices(m, n, k) * m * n * 4
        assert lib.xpuint8_linear_workspace_size(m, n, k) == want, (m, n, k)
    assert lib.xpuint8_linear_workspace_size(4, 32, 300) == -1
    assert lib.xpuint8_linear_workspace_size(4, 24, 512) == -1
    assert lib.xpuint8_linear_workspace_size(0, 32, 512) == -1


def test_ffn_workspace_size(lib):
    """The FFN's workspace: the bf16 [M, inner] activation rounded up to 256
    bytes, then one region that holds x quantized (row-major, then its fp32
    row scales from a 256-byte boundary) and afterwards the down-projection's
    linear workspace, whichever is larger; -1 for a shape or an activation the
    entry point rejects."""
    for m, inner, k in [(4096, 5120, 1280), (128, 5120, 1280), (1, 256, 256), (200, 1024, 512),
                        (4096, 10240, 2560), (64, 256, 4096)]:
        region = max(up256(m * k) + 4 * m, lib.xpuint8_linear_workspace_size(m, k, inner))
        for act in (3, 4, 5):
            assert lib.xpuint8_ffn_workspace_size(m, inner, k, act) == up256(2 * m * inner) + region
    assert lib.xpuint8_ffn_workspace_size(4, 512, 512, 2) == -1      # activation
    assert lib.xpuint8_ffn_workspace_size(4, 400, 512, 3) == -1      # inner % 256
    assert lib.xpuint8_ffn_workspace_size(4, 512, 300, 3) == -1      # K % 256
    assert lib.xpuint8_ffn_workspace_size(0, 512, 512, 3) == -1
