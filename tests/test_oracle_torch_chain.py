"""Pins for oracle/torch_chain.py, the torch-CPU restatement of
reference/convrot_linear.py that bench.py times as the CPU baseline:

* the Hadamard matrix is the numpy oracle's kron(H4,H4,H4,H4)/16 exactly;
* after the rotation, its quantize / _int_mm / dequant / bias steps equal the
  numpy restatement of the same reference lines (oracle.convrot_int8_linear)
  bit for bit on the same rotated input;
* its rotation (a BLAS matmul) agrees with the reference's op-ordered
  Hadamard to fp32 rounding, and the whole chain agrees with the GPU path's
  oracle (oracle.linear) within the north star's bf16 rel-err 1e-2.
"""

import numpy as np
import torch

import oracle as O
from oracle import torch_chain as TC


def _b(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _inputs(m=256, k=1280, n=512, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[:8]] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    w8, ws = O.prepare_weight(_b(w))
    return x, torch.from_numpy(w8), torch.from_numpy(ws), bias


def test_matrix_is_the_oracles():
    assert np.array_equal(TC.hadamard_matrix().double().numpy(), O.hadamard256_matrix())


def test_steps_after_the_rotation_match_the_numpy_restatement():
    x, w8, ws, bias = _inputs()
    xr = torch.from_numpy(O.hadamard256(O.bf16_to_f32(_b(x))))
    got = TC.quantized_linear_from_rotated(xr, w8, ws, bias)
    want = O.convrot_int8_linear(xr.numpy(), w8.numpy(), ws.numpy(), _b(bias))
    assert np.array_equal(_b(got), want)


def test_rotation_and_chain_agree_with_the_oracle():
    x, w8, ws, bias = _inputs(seed=1)
    h = TC.hadamard_matrix()
    xr = (x.float().reshape(-1, 5, 256) @ h).reshape(x.shape)
    ref = O.hadamard256(O.bf16_to_f32(_b(x)))
    assert np.max(np.abs(xr.numpy() - ref)) <= 4e-6 * np.abs(ref).max()
    got = O.bf16_to_f32(_b(TC.convrot_int8_linear(x, w8, ws, bias, h))).astype(np.float64)
    want = O.bf16_to_f32(O.linear(_b(x), w8.numpy(), ws.numpy(),
                                  O.bf16_to_f32(_b(bias)))).astype(np.float64)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-2
