"""Tensor-level API: torch.ops.paia_gemv.* custom ops (torch.library) backed by libpaia_gemv.so.

    from paia_gemv import ops
    y = ops.gemv_fp8(Wq, scale, x)                 # x bf16 [K] or [M,K] (M <= 16) -> y bf16 [N] or [M,N]
    ops.gemv_int4_zp(Wq, s, z, x, bias=b, out=y)   # writes y, allocates nothing

One activation row runs the M = 1 GEMV kernels (`variant` indexes GemvLib.variants / variants_fp8 / variants_int4);
M = 2..16 rows run the small-batch kernels, row-streaming or matrix-core (`variant` indexes
GemvLib.variants_batch[fmt]); -1 is the library's choice.

The ops are registered by libpaia_gemv_torch.so (csrc/torch_ops.cpp); they run on torch's current stream and are
HIP-graph capturable. There is no fallback: if the extension is missing, `load()` raises.
"""
from __future__ import annotations

import os
from pathlib import Path

import torch

_PKG_ROOT = Path(__file__).resolve().parent.parent
_loaded = None


def find_torch_ext() -> str:
    env = os.environ.get("PAIA_GEMV_TORCH_LIB")
    cands = ([env] if env else []) + [str(_PKG_ROOT / "build" / "libpaia_gemv_torch.so")]
    for c in cands:
        if c and os.path.exists(c):
            return c
    raise FileNotFoundError("libpaia_gemv_torch.so not found (run `python paia-project_amd/build.py`). Tried: "
                            + ", ".join(c for c in cands if c))


def load() -> str:
    """Load the torch extension once (it links libpaia_gemv.so from the same directory). Returns its path."""
    global _loaded
    if _loaded is None:
        path = find_torch_ext()
        torch.ops.load_library(path)
        _loaded = path
    return _loaded


def gemv_bf16(W, x, bias=None, variant=-1, out=None):
    load()
    if out is None:
        return torch.ops.paia_gemv.gemv_bf16(W, x, bias, variant)
    torch.ops.paia_gemv.gemv_bf16_out(W, x, bias, variant, out)
    return out


def gemv_fp8(Wq, scale, x, bias=None, variant=-1, out=None):
    load()
    if out is None:
        return torch.ops.paia_gemv.gemv_fp8(Wq, scale, x, bias, variant)
    torch.ops.paia_gemv.gemv_fp8_out(Wq, scale, x, bias, variant, out)
    return out


def gemv_int4(Wq, scales, x, variant=-1, out=None):
    """Reference INT4 format: Wq uint8 [N,K/2] (or int32 [N,K/8]), fp16 scales [N,K/128], zero point 8."""
    load()
    if out is None:
        return torch.ops.paia_gemv.gemv_int4(Wq, scales, x, variant)
    torch.ops.paia_gemv.gemv_int4_out(Wq, scales, x, variant, out)
    return out


def gemv_int4_zp(Wq, scales, zeros, x, bias=None, variant=-1, out=None):
    """Asymmetric INT4: bf16 scales [N,G], zeros uint8 [N,ceil(G/2)], optional bf16 bias [N]."""
    load()
    if out is None:
        return torch.ops.paia_gemv.gemv_int4_zp(Wq, scales, zeros, x, bias, variant)
    torch.ops.paia_gemv.gemv_int4_zp_out(Wq, scales, zeros, x, bias, variant, out)
    return out


def dequant_fp8(Wq, scale):
    load()
    return torch.ops.paia_gemv.dequant_fp8(Wq, scale)


def dequant_int4(Wq, scales):
    load()
    return torch.ops.paia_gemv.dequant_int4(Wq, scales)


def dequant_int4_zp(Wq, scales, zeros):
    load()
    return torch.ops.paia_gemv.dequant_int4_zp(Wq, scales, zeros)


def quantize_fp8_rowwise(W):
    """fp32 W [N,K] on the device -> (q uint8 e4m3 [N,K], scale fp32 [N]) by the HIP quantizer."""
    load()
    return torch.ops.paia_gemv.quantize_fp8_rowwise(W)


def quantize_int4_g128(W):
    """fp32 W [N,K] on the device -> (packed uint8 [N,K/2], scales fp16 [N,K/128]) by the HIP quantizer."""
    load()
    return torch.ops.paia_gemv.quantize_int4_g128(W)


def quantize_int4_zp_g128(W):
    """fp32 W [N,K] on the device -> asymmetric INT4 (packed [N,K/2], scales bf16 [N,G], zeros [N,ceil(G/2)])."""
    load()
    return torch.ops.paia_gemv.quantize_int4_zp_g128(W)
