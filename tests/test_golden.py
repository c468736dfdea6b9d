"""Known-answer vectors (tests/golden/convrot_known_answers.json, written by
tests/golden/make_golden.py from closed forms and exact integer arithmetic)
against the CPU oracle and, on a GPU, the library."""

import json
import os

import numpy as np
import pytest

import oracle as O

with open(os.path.join(os.path.dirname(__file__), "golden", "convrot_known_answers.json")) as _f:
    G = json.load(_f)


def _u16(v):
    return np.asarray(v, dtype=np.uint16)


def _f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


def hadamard_signs():
    bits = np.unpackbits(np.frombuffer(bytes.fromhex(G["hadamard_signs"]["hex"]), np.uint8))
    return np.where(bits.reshape(256, 256) == 1, -1.0, 1.0)


# --------------------------------------------------------------------- oracle
def test_oracle_hadamard_is_the_golden_matrix():
    assert np.array_equal(O.hadamard256_matrix(), hadamard_signs() / 16.0)
    # and the transform applied to every unit vector
    eye = np.eye(256, dtype=np.float32)
    assert np.array_equal(O.hadamard256(eye).T.astype(np.float64), hadamard_signs() / 16.0)


def test_oracle_quantize_row_ties():
    t = G["quantize_row_ties"]
    q, s = O.quantize_row(_u16(t["x_bf16"])[None, :])
    assert q[0].tolist() == t["q"] and s.view(np.uint32)[0] == t["scale_f32"]


@pytest.mark.parametrize("i", range(4))
def test_oracle_convrot_rows(i):
    r = G["convrot_rows"][i]
    q, s = O.convrot_quantize(_u16(r["x_bf16"])[None, :])
    assert q[0].tolist() == r["q"], r["name"]
    assert s.view(np.uint32)[0] == r["scale_f32"], r["name"]


def test_oracle_int_mm_and_dequant():
    t = G["int_mm"]
    got = O.int_mm(np.array(t["a"], np.int8), np.array(t["b"], np.int8))
    assert got.tolist() == t["acc"]
    d = G["dequant"]
    out = O.dequant(np.array(d["acc"], np.int32), np.array(d["x_scale"], np.float32),
                    np.array(d["w_scale"], np.float32), np.array(d["bias"], np.float32))
    assert out.tolist() == d["out_bf16"]


def test_oracle_rotate_spikes():
    for sp in G["rotate_spikes"]:
        assert O.rotate_bf16(_u16(sp["x_bf16"])[None, :])[0].tolist() == sp["out_bf16"]


# ------------------------------------------------------------------- library
@pytest.mark.gpu
def test_library_on_the_golden_vectors(dev):
    import torch
    from gpu_util import from_bits, npy, bits
    from xpu_kernels import int8
    t = G["quantize_row_ties"]
    q, s = int8.quantize_row(from_bits(_u16(t["x_bf16"])[None, :], dev))
    assert npy(q)[0].tolist() == t["q"] and npy(s).view(np.uint32)[0] == t["scale_f32"]
    for r in G["convrot_rows"]:
        q, s = int8.quantize(from_bits(_u16(r["x_bf16"])[None, :], dev))
        assert npy(q)[0].tolist() == r["q"], r["name"]
        assert npy(s).view(np.uint32)[0] == r["scale_f32"], r["name"]
    for sp in G["rotate_spikes"]:
        y = int8.rotate(from_bits(_u16(sp["x_bf16"])[None, :], dev))
        assert bits(y)[0].tolist() == sp["out_bf16"]
    m = G["int_mm"]
    a = torch.tensor(m["a"], dtype=torch.int8)
    b = torch.tensor(m["b"], dtype=torch.int8)
    # the GEMM's shape contract (K, N multiples of 16): pad with zero columns/rows
    ap = torch.zeros((5, 64), dtype=torch.int8); ap[:, :] = a
    bp = torch.zeros((16, 64), dtype=torch.int8); bp[:7] = b
    acc = npy(int8.int_mm(ap.to(dev), bp.to(dev).t()))
    assert acc[:, :7].tolist() == m["acc"]
