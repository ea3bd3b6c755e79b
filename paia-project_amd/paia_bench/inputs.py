"""Seeded synthetic operands for the BASELINE configurations, generated on the CPU so a CPU check sees identical bits.

Seed convention: torch.Generator().manual_seed(1000 + N + K) (paia-bench/bench/ops/ours_bf16.py:70, on the CPU here),
draws in the order listed per format:
  bf16    W = bf16(0.02 * randn(N,K)); x = bf16(randn(K))
  fp8     W = 0.02 * randn(N,K) quantised with quantize_fp8_rowwise (e4m3fn, scale = amax/448); x = bf16(randn(K))
  int4    W = 0.02 * randn(N,K) quantised with quantize_int4_g128 (the reference format); x = bf16(randn(K))
  int4zp  q = randint(0,16,(N,K)); s = bf16(U[0.001,0.01]) [N,G]; z = randint(0,16,(N,G)); x = bf16(randn(K))
  bias    b = bf16(0.02 * randn(N)) (drawn last, only when asked)
Arrays are returned as numpy bit patterns (uint16 for bf16/fp16, uint8 for codes) plus torch CPU tensors.
"""
from __future__ import annotations

import numpy as np
import torch

from paia_gemv import quant


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16) if t.element_size() == 2 else t.numpy()


def make_operands(fmt: str, N: int, K: int, bias: bool = False, seed: int | None = None) -> dict:
    """Operands for one GEMV as CPU torch tensors: keys W/Wq, scale(s), zeros, x, bias (bf16 tensors for bf16 data)."""
    g = torch.Generator().manual_seed(1000 + N + K if seed is None else seed)
    out: dict = {"fmt": fmt, "N": N, "K": K}
    if fmt == "bf16":
        out["W"] = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16)
    elif fmt == "fp8":
        W = 0.02 * torch.randn(N, K, generator=g)
        out["Wq"], out["scale"] = quant.quantize_fp8_rowwise(W)
    elif fmt == "int4":
        W = 0.02 * torch.randn(N, K, generator=g)
        out["Wq"], out["scales"] = quant.quantize_int4_g128(W)
    elif fmt == "int4zp":
        G = K // 128
        q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
        s = (0.001 + 0.009 * torch.rand(N, G, generator=g)).to(torch.bfloat16)
        z = torch.randint(0, 16, (N, G), generator=g, dtype=torch.uint8)
        out["Wq"], out["scales"], out["zeros"] = quant.pack_int4(q), s, quant.pack_zeros(z)
    else:
        raise ValueError(fmt)
    out["x"] = torch.randn(K, generator=g).to(torch.bfloat16)
    out["bias"] = (0.02 * torch.randn(N, generator=g)).to(torch.bfloat16) if bias else None
    return out


def as_numpy(ops: dict) -> dict:
    """Bit-pattern numpy views of make_operands() output (for the CPU oracle)."""
    res = {}
    for k, v in ops.items():
        if isinstance(v, torch.Tensor):
            res[k] = _bits(v)
        else:
            res[k] = v
    return res


def to_device(ops: dict, device="cuda") -> dict:
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ops.items()}
