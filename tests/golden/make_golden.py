#!/usr/bin/env python3
"""Writes tests/golden/convrot_known_answers.json: known-answer vectors for the
ConvRot INT8 path, computed from closed forms and exact integer arithmetic
only (never from the oracle or the library they check).

    python tests/golden/make_golden.py

Contents
* ``hadamard_signs``: the 256x256 group transform H = kron(H4,H4,H4,H4)/16 as
  sign bits (entry (i, j) is +1/16 or -1/16), built digit by digit from
  H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]
  (okolenmi/oko-xpu-kernels src/xpuint8.cpp:55-75) with i = sum 4^d i_d.
* ``quantize_row_ties``: the reference's tie known answer
  (tests/test_quantize.py:85-91): [127, 254, -254, 63] -> [64, 127, -127, 32],
  scale 2.0.
* ``convrot_rows``: rows with a closed-form ConvRot quantization
  - zero row: scale 1e-30, codes 0;
  - constant row c: the all-ones vector is a fixed point of H (every row of
    H4/2 sums to 1), so the rotated row is c and every code is 127 with
    scale c/127;
  - a single spike v at position j of a group: the rotated group is
    (v/16) * H[:, j] (signs +-1), every code of that group is +-127, the other
    groups are 0, scale (|v|/16)/127.
* ``int_mm``: a small int8 x int8^T product in exact int64 (brute force).
* ``dequant``: accumulators with power-of-two scales and a bias whose fp32
  results are exact, so their bf16 roundings are fixed.
* ``rotate_spikes``: bf16 rotations of power-of-two spikes (exact: +-v/16).
"""

import json
import os

import numpy as np

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.int64)


def hadamard_signs():
    """Sign of H[i, j] = prod over the four base-4 digits of H4[i_d, j_d]."""
    s = np.ones((256, 256), dtype=np.int64)
    i = np.arange(256)
    for d in range(4):
        di = (i >> (2 * d)) & 3
        s *= H4[di[:, None], di[None, :]]
    return s


def f32_bits(x):
    return int(np.array(x, dtype=np.float32).view(np.uint32))


def bf16_bits_exact(x):
    """bf16 bits of a value that is exactly representable in bf16."""
    u = int(np.array(x, dtype=np.float32).view(np.uint32))
    assert u & 0xFFFF == 0, x
    return u >> 16


def main():
    out = {}
    s = hadamard_signs()
    out["hadamard_signs"] = {
        "doc": "row-major 256x256, bit 1 = -1/16, bit 0 = +1/16; packed 8 per byte, MSB first",
        "hex": np.packbits((s < 0).astype(np.uint8).reshape(-1)).tobytes().hex(),
    }
    out["quantize_row_ties"] = {
        "x_bf16": [bf16_bits_exact(v) for v in (127.0, 254.0, -254.0, 63.0)],
        "q": [64, 127, -127, 32],
        "scale_f32": f32_bits(2.0),
    }

    rows = []
    k = 512
    rows.append({"name": "zero", "x_bf16": [0] * k, "q": [0] * k, "scale_f32": f32_bits(1e-30)})
    c = 3.0
    sc = np.float32(np.float32(c) / np.float32(127.0))
    rows.append({"name": "constant 3.0", "x_bf16": [bf16_bits_exact(c)] * k, "q": [127] * k,
                 "scale_f32": f32_bits(sc)})
    for (g, j, v) in ((0, 5, 2.0), (1, 200, -8.0)):
        x = [0] * k
        x[256 * g + j] = bf16_bits_exact(v)
        q = [0] * k
        col = s[:, j] * (1 if v > 0 else -1)
        q[256 * g:256 * g + 256] = [int(127 * t) for t in col]
        rows.append({"name": f"spike {v} at group {g} position {j}", "x_bf16": x, "q": q,
                     "scale_f32": f32_bits(np.float32(np.float32(abs(v) / 16.0) / np.float32(127.0)))})
    out["convrot_rows"] = rows

    rng = np.random.default_rng(2024)
    a = rng.integers(-127, 128, (5, 64), dtype=np.int64)
    b = rng.integers(-127, 128, (7, 64), dtype=np.int64)
    acc = [[int(sum(int(a[m, t]) * int(b[n, t]) for t in range(64))) for n in range(7)] for m in range(5)]
    out["int_mm"] = {"a": a.tolist(), "b": b.tolist(), "acc": acc}

    # dequant: acc * (ws * xs) + bias with power-of-two scales: exact in fp32,
    # and each result chosen representable in bf16
    acc_d = [[3, -5, 12, 0], [96, -1, 7, 64]]
    xs = [0.5, 0.25]
    ws = [0.125, 2.0, 0.5, 1.0]
    bias = [1.0, -0.5, 0.0, 4.0]
    res = [[acc_d[m][n] * (ws[n] * xs[m]) + bias[n] for n in range(4)] for m in range(2)]
    out["dequant"] = {"acc": acc_d, "x_scale": xs, "w_scale": ws, "bias": bias,
                      "out_bf16": [[bf16_bits_exact(v) for v in r] for r in res]}

    spikes = []
    for (j, v) in ((0, 1.0), (37, -4.0), (255, 0.5)):
        x = [0] * 256
        x[j] = bf16_bits_exact(v)
        y = [bf16_bits_exact(float(v) / 16.0 * float(t)) for t in s[:, j]]
        spikes.append({"x_bf16": x, "out_bf16": y})
    out["rotate_spikes"] = spikes

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "convrot_known_answers.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
