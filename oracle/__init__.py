"""CPU oracle for the ConvRot INT8 linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference library's
ConvRot INT8 path (the SYCL kernels in ``src/xpuint8.cpp``, the torch chains in
``python/xpu_kernels/int8/ops.py`` and the oracle ``reference/convrot_linear.py``
of okolenmi/oko-xpu-kernels).  Every function cites the reference file:line it
follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the thing timed on the CPU).  The product path -- the HIP library
and the ``xpu_kernels`` package -- never imports or calls it.

Pinning status of each function (how a plausible mistake would be caught) is
listed in ``PINNING`` below and exercised by ``tests/test_oracle_*.py``.
"""

from .convrot import *  # noqa: F401,F403
from .convrot import __all__ as _convrot_all
from .activations import *  # noqa: F401,F403
from .activations import __all__ as _act_all
from .rope import *  # noqa: F401,F403
from .rope import __all__ as _rope_all

__all__ = list(_convrot_all) + list(_act_all) + list(_rope_all)

#: function -> the independent checks that pin it (tests/test_oracle_*.py)
PINNING = {
    "hadamard256": "explicit kron(H4,H4,H4,H4)/16 matrix in float64; all-ones fixed "
                   "point; H e_j = +-1/16 with the kron signs; involution; norm; "
                   "literal lane-per-group restatement of the reference loops",
    "rotate_bf16": "hadamard256 + bf16 RNE (bf16 rounding pinned against torch)",
    "convrot_quantize": "float64 formula (reference tests/test_quantize.py:42-52 "
                        "style); constant-row and zero-row known answers; "
                        "division-chain agreement (<=1e-4 tie flips)",
    "quantize_row": "float64 formula; tie known-answer [127,254,-254,63]->[64,127,-127,32] "
                    "(reference tests/test_quantize.py:85-91); torch chain",
    "prepare_weight": "torch chain of ops.py:93-99 on CPU; float64 formula",
    "int_mm": "torch._int_mm on CPU; brute-force int64 on small inputs",
    "dequant": "float64 closed form within 1 bf16 ulp; bias/no-bias",
    "gelu_erf_f32": "torch F.gelu(approximate='none') over all 65536 bf16 inputs "
                    "(mismatches bounded, each <=1 bf16 ulp); float64 closed form",
    "linear": "composition; float64 x@W.T within INT8 error; "
              "reference convrot_linear.py restatement (<=1e-4 code flips)",
    "dequant_weight": "torch chain (w8.float()*s).bf16 then the pinned rotation; "
                      "round trip to W within the int8 step",
    "linear_dx_int8": "torch chain of ops.py:366-377 (bf16 mul, torch._int_mm); "
                      "float64 dy@W within INT8 error",
    "linear_dw": "torch float64 matmul",
    "column_sum": "float64 exact sums within the float32 chunked-summation bound before "
                  "the one bf16 rounding; closed forms (constant columns sum to M*v, "
                  "+v/-v pairs to zero); torch's dy.sum(0) on bf16 within one bf16 ulp",
    "linear_dx": "torch float64 matmul dy @ w; transposed-operand identity with linear_dw",
    "activate": "torch bf16 eager chains (gelu_tanh, silu*u, situ, h*gelu(g), gelu) "
                "within 1 bf16 ulp on <0.5% of elements; float64 closed forms "
                "(test_oracle_activations); tanh_fast vs float64 tanh on all bf16",
    "quantize_act": "convrot_quantize of the torch chain's activation, bit for bit "
                    "on rows where the activations agree",
    "dequant_act / dequant_act_quantize": "torch chain bf16(acc*(ws*xs)) then the "
                                          "activation; quantize of it on equal rows",
    "ffn": "float64 down(geglu(up(x)))+b with the unquantized weights",
    "rms_rope_dequant / rms_rope_bf16": "float64 closed forms: identity rotation gives "
                                        "x/rms(x)*scale; a constant row gives +-1; a pair "
                                        "(1, 1) rotated by theta gives (cos-sin, sin+cos); "
                                        "the rotation keeps each pair's norm; split-half and "
                                        "interleaved agree under the dim permutation",
}
