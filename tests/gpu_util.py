"""Helpers for the GPU parity tests: run one GEMV through the C ABI on seeded operands and fetch bit patterns."""
import functools
import sys

import numpy as np
import torch

from paia_bench.inputs import as_numpy, make_operands


def note(msg: str) -> None:
    """Name the case on the real stdout before a GPU step (survives pytest's capture if the process dies)."""
    sys.__stdout__.write(f"    [case] {msg}\n")
    sys.__stdout__.flush()


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).ravel()


def nan_filled(N, device):
    return torch.full((N,), float("nan"), dtype=torch.bfloat16, device=device)


def run_gemv(lib, fmt, dev_ops, variant, y=None, mode="fused", scratch=None, stream=None):
    """Launch one GEMV on device operands (dict from paia_bench.inputs.to_device). Returns y (bf16 [N])."""
    N, K = dev_ops["N"], dev_ops["K"]
    x = dev_ops["x"]
    if y is None:
        y = nan_filled(N, x.device)
    b = dev_ops.get("bias")
    bp = b.data_ptr() if b is not None else None
    if fmt == "bf16":
        if bp is None:
            lib.bf16(dev_ops["W"].data_ptr(), x.data_ptr(), y.data_ptr(), N, K, variant, stream)
        else:
            lib.bf16_bias(dev_ops["W"].data_ptr(), x.data_ptr(), bp, y.data_ptr(), N, K, variant, stream)
    elif fmt == "fp8":
        if bp is None:
            lib.fp8(dev_ops["Wq"].data_ptr(), dev_ops["scale"].data_ptr(), x.data_ptr(), y.data_ptr(), N, K, variant,
                    stream)
        else:
            lib.fp8_bias(dev_ops["Wq"].data_ptr(), dev_ops["scale"].data_ptr(), x.data_ptr(), bp, y.data_ptr(), N, K,
                         variant, stream)
    elif fmt == "int4":
        args = (dev_ops["Wq"].data_ptr(), dev_ops["scales"].data_ptr(), x.data_ptr(), y.data_ptr())
        if mode == "fused":
            lib.int4(*args, N, K, variant, stream)
        elif mode == "naive":
            lib.int4_naive(*args, N, K, stream)
        else:
            lib.int4_unfused(*args, scratch.data_ptr(), N, K, stream)
    elif fmt == "int4zp":
        lib.int4_zp(dev_ops["Wq"].data_ptr(), dev_ops["scales"].data_ptr(), dev_ops["zeros"].data_ptr(), x.data_ptr(),
                    bp, y.data_ptr(), N, K, variant, stream)
    else:
        raise ValueError(fmt)
    return y


def oracle_ref(O, fmt, np_ops, rows=None):
    """fp64 oracle output (and the fp32-matmul reference when rows is None) for the operands."""
    b = np_ops.get("bias")
    if fmt == "bf16":
        ref64 = O.gemv_bf16_f64(np_ops["W"], np_ops["x"], b, rows)
    elif fmt == "fp8":
        ref64 = O.gemv_fp8_f64(np_ops["Wq"], np_ops["scale"], np_ops["x"], b, rows)
    elif fmt == "int4":
        ref64 = O.gemv_int4_f64(np_ops["Wq"], np_ops["scales"], np_ops["x"], rows)
    else:
        ref64 = O.gemv_int4_zp_f64(np_ops["Wq"], np_ops["scales"], np_ops["zeros"], np_ops["x"], b, rows)
    return ref64


def dequant_oracle(O, fmt, np_ops):
    if fmt == "bf16":
        return O.bf16_bits_to_f32(np_ops["W"]).reshape(np_ops["W"].shape)
    if fmt == "fp8":
        return O.dequant_fp8(np_ops["Wq"], np_ops["scale"])
    if fmt == "int4":
        return O.dequant_int4(np_ops["Wq"], np_ops["scales"])
    return O.dequant_int4_zp(np_ops["Wq"], np_ops["scales"], np_ops["zeros"])


@functools.lru_cache(maxsize=48)
def _make_cached(fmt, N, K, bias, seed):
    ops = make_operands(fmt, N, K, bias=bias, seed=seed)
    return ops, as_numpy(ops)


def make(fmt, N, K, bias=False, seed=None):
    """Seeded CPU operands (torch tensors, numpy bit patterns), memoised across tests; callers get fresh dicts."""
    ops, np_ops = _make_cached(fmt, N, K, bias, seed)
    return dict(ops), dict(np_ops)
