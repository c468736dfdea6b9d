"""``xpu_kernels.int8.selftest()``: does the library work on this machine?

The counterpart of the reference's ``python/xpu_kernels/int8/selftest.py:37-184``:
the pieces checked against each other on the device -- weight preparation, the
accumulator path against the fused linear, the strided slice, the fused GEGLU
FFN against its unfused chain, the backward pieces -- and the INT8 result
against a bf16 GEMM.  Not the parity suite (that lives in the repository's
``tests/``, against the CPU oracle).
"""

from __future__ import annotations

import torch

from . import _lib as L
from ._lib import available, device_name


def selftest(verbose: bool = True) -> bool:
    from .ops import (dequant, dequant_act_quantize, dequant_slice, dequant_weight,
                      dequant_weight_torch, ffn, int_mm, linear, linear_acc, linear_dx_int8,
                      prepare_weight, quantize, quantize_row, quantize_row_torch)

    if not available():
        if verbose:
            print(f"libxpuint8 unavailable: {L._ERR}")
        return False
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator(device="cpu").manual_seed(0)
    M, K, N = 512, 1024, 512

    def rnd(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).to(torch.bfloat16).to(dev)

    x, w = rnd(M, K, s=0.5), rnd(N, K, s=0.05)
    bias = (torch.randn(N, generator=g) * 0.1).to(dev)
    w8, ws = prepare_weight(w)
    y = linear(x, w8, ws, bias)
    ref = (x.float() @ w.float().t() + bias).to(torch.bfloat16)
    rel = ((y.float() - ref.float()).norm() / ref.float().norm()).item()

    acc, xs = linear_acc(x, w8, ws)
    same = dequant(acc, xs, ws, bias).view(torch.int16).equal(y.view(torch.int16))

    acc_w, xs_w = linear_acc(x, torch.cat([w8, w8], 0), torch.cat([ws, ws]))
    sl = dequant_slice(acc_w[:, :N], xs_w, ws, bias)
    slice_same = sl.view(torch.int16).equal(dequant(acc_w[:, :N].contiguous(), xs_w, ws,
                                                    bias).view(torch.int16))

    kff = 1024
    wup8, wup_s = prepare_weight(rnd(2 * kff, K, s=0.05))
    wdn8, wdn_s = prepare_weight(rnd(K, kff, s=0.05))
    xup = rnd(M, K, s=0.5)
    out = ffn(xup, wup8, wup_s, wdn8, wdn_s, act="geglu_erf")
    acc2, xs2 = linear_acc(xup, wup8, wup_s)
    d = dequant(acc2, xs2, wup_s)
    hidden, gate = d.chunk(2, dim=-1)
    q2, s2 = quantize(hidden * torch.nn.functional.gelu(gate))
    q2f, s2f = dequant_act_quantize(acc2, xs2, wup_s, "geglu_erf")
    fused_q_same = q2f.equal(q2) and s2f.view(torch.int32).equal(s2.view(torch.int32))
    chain = dequant(int_mm(q2f, wdn8.t()), s2f, wdn_s)
    ffn_same = out.view(torch.int16).equal(chain.view(torch.int16))

    dy = rnd(M, N, s=0.5)
    q_f, s_f = quantize_row(dy)
    # the torch chain on the CPU: its scalar division is correctly rounded
    # there (ROCm's GPU division is not, so on the device it agrees to +-1)
    q_c, s_c = quantize_row_torch(dy.cpu())
    rowq_same = q_f.cpu().equal(q_c) and s_f.cpu().view(torch.int32).equal(s_c.view(torch.int32))
    deq_same = dequant_weight(w8, ws).view(torch.int16).equal(
        dequant_weight_torch(w8, ws).view(torch.int16))
    xr = x.detach().float().requires_grad_(True)
    torch.nn.functional.linear(xr, w.float()).backward(dy.float())
    dx_q = linear_dx_int8(dy, w8, ws)
    dx_rel = ((dx_q.float() - xr.grad).norm() / xr.grad.norm()).item()

    ok = (rel < 0.02 and same and slice_same and ffn_same and rowq_same and deq_same
          and dx_rel < 0.04)
    if verbose:
        print(f"device             : {device_name()}")
        print(f"INT8 vs bf16       : relative error {rel:.4f} (expect < 0.02)")
        print(f"acc path == linear : {same}")
        print(f"strided slice      : {slice_same}")
        print(f"fused dequant+GEGLU+quantize == chain codes: {fused_q_same} "
              f"(GELU: the build's exact table vs torch's erf may differ in a few bf16 "
              f"values below -3)")
        print(f"GEGLU FFN == chain through int_mm: {ffn_same}")
        print(f"quantize_row == torch chain (CPU): {rowq_same}")
        print(f"dequant_weight == torch chain: {deq_same}")
        print(f"dx (int8 weight) vs fp32 autograd: rel {dx_rel:.4f} (expect < 0.04)")
        print("PASS" if ok else "FAIL")
    return ok
