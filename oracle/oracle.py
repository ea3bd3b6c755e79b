"""CPU oracle for the PAIA GEMV family -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the checker
(or, for cpu_baseline, as the CPU path being timed beside the GPU). The paia_gemv package never imports it.

It wraps oracle/libpaia_oracle.so (the C restatement in paia_oracle.c, built by oracle/Makefile) with numpy arrays,
and adds the fp32 matmul reference the reference harness uses (x.float() @ Wdeq.t(), paia-bench/bench/ops/
ours_quant.py:69-71, cublas_bf16.py:33-38). Each wrapper names the reference lines the C function follows in its
docstring there.

Optional: when oracle/_ref/libquant_host_ref.so exists (the reference's own quant_host.h compiled in place by
oracle/Makefile), `ref_lib()` returns it so tests can compare the restatement against the reference itself.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB_PATH = HERE / "libpaia_oracle.so"
_REF_PATH = HERE / "_ref" / "libquant_host_ref.so"

_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_int = ctypes.c_int

_lib = None
_ref = None


def build(force: bool = False) -> Path:
    """Compile libpaia_oracle.so with oracle/Makefile (gcc). Returns its path."""
    if force or not _LIB_PATH.exists() or _LIB_PATH.stat().st_mtime < (HERE / "paia_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.po_e4m3_to_f32.restype = ctypes.c_float
        L.po_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.po_f32_to_e4m3.restype = ctypes.c_uint8
        L.po_f32_to_e4m3.argtypes = [ctypes.c_float]
        L.po_f32_to_f16.restype = ctypes.c_uint16
        L.po_f32_to_f16.argtypes = [ctypes.c_float]
        L.po_f16_to_f32.restype = ctypes.c_float
        L.po_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.po_f32_to_bf16.restype = ctypes.c_uint16
        L.po_f32_to_bf16.argtypes = [ctypes.c_float]
        L.po_bf16_to_f32.restype = ctypes.c_float
        L.po_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.po_quantize_fp8_rowwise.argtypes = [_f32p, _int, _int, _u8p, _f32p]
        L.po_quantize_int4_g128.argtypes = [_f32p, _int, _int, _u8p, _u16p]
        L.po_quantize_int4_zp_g128.argtypes = [_f32p, _int, _int, _u8p, _u16p, _u8p]
        L.po_dequant_fp8.argtypes = [_u8p, _f32p, _int, _int, _f32p]
        L.po_dequant_int4.argtypes = [_u8p, _u16p, _int, _int, _f32p]
        L.po_dequant_int4_zp.argtypes = [_u8p, _u16p, _u8p, _int, _int, _f32p]
        L.po_dequant_int4_bf16.argtypes = [_u8p, _u16p, _int, _int, _u16p]
        L.po_gemv_f64.argtypes = [_f32p, _u16p, _vp, _int, _int, _vp, _int, _f64p]
        L.po_gemv_f32.argtypes = [_f32p, _u16p, _vp, _int, _int, _vp, _int, _f32p]
        L.po_gemv_bf16_f64.argtypes = [_u16p, _u16p, _vp, _int, _int, _vp, _int, _f64p]
        L.po_gemv_fp8_f64.argtypes = [_u8p, _f32p, _u16p, _vp, _int, _int, _vp, _int, _f64p]
        L.po_gemv_int4_f64.argtypes = [_u8p, _u16p, _u16p, _int, _int, _vp, _int, _f64p]
        L.po_gemv_int4_zp_f64.argtypes = [_u8p, _u16p, _u8p, _u16p, _vp, _int, _int, _vp, _int, _f64p]
        _lib = L
    return _lib


def ref_lib():
    """The reference's own quant_host.h compiled in place (oracle/_ref), or None where it was not built."""
    global _ref
    if _ref is None and _REF_PATH.exists():
        R = ctypes.CDLL(str(_REF_PATH))
        R.ref_e4m3_decode.restype = ctypes.c_float
        R.ref_e4m3_decode.argtypes = [ctypes.c_uint8]
        R.ref_e4m3_encode.restype = ctypes.c_uint8
        R.ref_e4m3_encode.argtypes = [ctypes.c_float]
        R.ref_f32_to_f16_bits.restype = ctypes.c_uint16
        R.ref_f32_to_f16_bits.argtypes = [ctypes.c_float]
        R.ref_f16_bits_to_f32.restype = ctypes.c_float
        R.ref_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        R.ref_quantize_fp8_rowwise.argtypes = [_f32p, _int, _int, _u8p, _f32p]
        R.ref_dequant_fp8.argtypes = [_u8p, _f32p, _int, _int, _f32p]
        R.ref_quantize_int4_g128.argtypes = [_f32p, _int, _int, _u8p, _u16p]
        R.ref_dequant_int4.argtypes = [_u8p, _u16p, _int, _int, _f32p]
        _ref = R
    return _ref


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _opt_ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _rows_arg(rows):
    if rows is None:
        return None, 0, None
    r = _c(rows, np.int32)
    return r, len(r), r.ctypes.data_as(_vp)


# ---------------------------------------------------------------------------------------------------------------
# scalar formats (vectorised over arrays)
# ---------------------------------------------------------------------------------------------------------------

def e4m3_table() -> np.ndarray:
    """float32[256]: the value of every e4m3fn code (NaN for 0x7F/0xFF). quant_host.h:18-23."""
    L = lib()
    return np.array([L.po_e4m3_to_f32(c) for c in range(256)], dtype=np.float32)


def e4m3_encode(v) -> np.ndarray:
    L = lib()
    v = np.asarray(v, dtype=np.float32).ravel()
    return np.array([L.po_f32_to_e4m3(float(x)) for x in v], dtype=np.uint8)


def f32_to_f16_bits(v) -> np.ndarray:
    L = lib()
    v = np.asarray(v, dtype=np.float32).ravel()
    return np.array([L.po_f32_to_f16(float(x)) for x in v], dtype=np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    L = lib()
    h = np.asarray(h, dtype=np.uint16).ravel()
    return np.array([L.po_f16_to_f32(int(x)) for x in h], dtype=np.float32)


def f32_to_bf16_bits(v) -> np.ndarray:
    """Vectorised RNE float32 -> bf16 bits (emulate_formats.py:26-28), identical to po_f32_to_bf16."""
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    out = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ---------------------------------------------------------------------------------------------------------------
# quantizers / dequantizers
# ---------------------------------------------------------------------------------------------------------------

def quantize_fp8_rowwise(W):
    """W fp32 [N,K] -> (q uint8 [N,K], scale fp32 [N]). quant.py:8-13 / quant_host.h:73-81."""
    W = _c(W, np.float32)
    N, K = W.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    lib().po_quantize_fp8_rowwise(W, N, K, q, s)
    return q, s


def quantize_int4_g128(W):
    """W fp32 [N,K] -> (packed uint8 [N,K/2], scales fp16 bits uint16 [N,K/128]). quant.py:20-31."""
    W = _c(W, np.float32)
    N, K = W.shape
    assert K % 128 == 0
    p = np.empty((N, K // 2), np.uint8)
    s = np.empty((N, K // 128), np.uint16)
    lib().po_quantize_int4_g128(W, N, K, p, s)
    return p, s


def quantize_int4_zp_g128(W):
    """W fp32 [N,K] -> asymmetric INT4 (packed uint8 [N,K/2], scales bf16 bits uint16 [N,G], zeros uint8
    [N,ceil(G/2)]). No reference code: the closed form of paia_oracle.c, pinned by tests/test_oracle.py."""
    W = _c(W, np.float32)
    N, K = W.shape
    assert K % 128 == 0
    G = K // 128
    p = np.empty((N, K // 2), np.uint8)
    s = np.empty((N, G), np.uint16)
    z = np.empty((N, (G + 1) // 2), np.uint8)
    lib().po_quantize_int4_zp_g128(W, N, K, p, s, z)
    return p, s, z


def dequant_fp8(q, scale):
    q = _c(q, np.uint8)
    N, K = q.shape
    out = np.empty((N, K), np.float32)
    lib().po_dequant_fp8(q, _c(scale, np.float32), N, K, out)
    return out


def dequant_int4(packed, scales_f16):
    packed = _c(packed, np.uint8)
    N, half = packed.shape
    out = np.empty((N, 2 * half), np.float32)
    lib().po_dequant_int4(packed, _c(scales_f16, np.uint16), N, 2 * half, out)
    return out


def dequant_int4_zp(packed, scales_bf16, zeros):
    packed = _c(packed, np.uint8)
    N, half = packed.shape
    out = np.empty((N, 2 * half), np.float32)
    lib().po_dequant_int4_zp(packed, _c(scales_bf16, np.uint16), _c(zeros, np.uint8), N, 2 * half, out)
    return out


def dequant_int4_bf16(packed, scales_f16):
    packed = _c(packed, np.uint8)
    N, half = packed.shape
    out = np.empty((N, 2 * half), np.uint16)
    lib().po_dequant_int4_bf16(packed, _c(scales_f16, np.uint16), N, 2 * half, out)
    return out


# ---------------------------------------------------------------------------------------------------------------
# GEMV references
# ---------------------------------------------------------------------------------------------------------------

def gemv_f64(Wd, x_bf16, bias_bf16=None, rows=None):
    Wd = _c(Wd, np.float32)
    N, K = Wd.shape
    r, nr, rp = _rows_arg(rows)
    b = None if bias_bf16 is None else _c(bias_bf16, np.uint16)
    y = np.empty(nr if rows is not None else N, np.float64)
    lib().po_gemv_f64(Wd, _c(x_bf16, np.uint16), _opt_ptr(b), N, K, rp, nr, y)
    return y


def gemv_f32_seq(Wd, x_bf16, bias_bf16=None, rows=None):
    Wd = _c(Wd, np.float32)
    N, K = Wd.shape
    r, nr, rp = _rows_arg(rows)
    b = None if bias_bf16 is None else _c(bias_bf16, np.uint16)
    y = np.empty(nr if rows is not None else N, np.float32)
    lib().po_gemv_f32(Wd, _c(x_bf16, np.uint16), _opt_ptr(b), N, K, rp, nr, y)
    return y


def gemv_bf16_f64(W_bf16, x_bf16, bias_bf16=None, rows=None):
    W = _c(W_bf16, np.uint16)
    N, K = W.shape
    r, nr, rp = _rows_arg(rows)
    b = None if bias_bf16 is None else _c(bias_bf16, np.uint16)
    y = np.empty(nr if rows is not None else N, np.float64)
    lib().po_gemv_bf16_f64(W, _c(x_bf16, np.uint16), _opt_ptr(b), N, K, rp, nr, y)
    return y


def gemv_fp8_f64(q, scale, x_bf16, bias_bf16=None, rows=None):
    q = _c(q, np.uint8)
    N, K = q.shape
    r, nr, rp = _rows_arg(rows)
    b = None if bias_bf16 is None else _c(bias_bf16, np.uint16)
    y = np.empty(nr if rows is not None else N, np.float64)
    lib().po_gemv_fp8_f64(q, _c(scale, np.float32), _c(x_bf16, np.uint16), _opt_ptr(b), N, K, rp, nr, y)
    return y


def gemv_int4_f64(packed, scales_f16, x_bf16, rows=None):
    packed = _c(packed, np.uint8)
    N, half = packed.shape
    r, nr, rp = _rows_arg(rows)
    y = np.empty(nr if rows is not None else N, np.float64)
    lib().po_gemv_int4_f64(packed, _c(scales_f16, np.uint16), _c(x_bf16, np.uint16), N, 2 * half, rp, nr, y)
    return y


def gemv_int4_zp_f64(packed, scales_bf16, zeros, x_bf16, bias_bf16=None, rows=None):
    packed = _c(packed, np.uint8)
    N, half = packed.shape
    r, nr, rp = _rows_arg(rows)
    b = None if bias_bf16 is None else _c(bias_bf16, np.uint16)
    y = np.empty(nr if rows is not None else N, np.float64)
    lib().po_gemv_int4_zp_f64(packed, _c(scales_bf16, np.uint16), _c(zeros, np.uint8), _c(x_bf16, np.uint16),
                              _opt_ptr(b), N, 2 * half, rp, nr, y)
    return y


def gemv_f32_matmul(Wd, x_bf16, bias_bf16=None):
    """The reference harness's CPU path: fp32 matmul x.float() @ Wdeq.t() (+ bias), as numpy BLAS."""
    x = bf16_bits_to_f32(x_bf16)
    y = np.asarray(_c(Wd, np.float32) @ x, dtype=np.float32)
    if bias_bf16 is not None:
        y = y + bf16_bits_to_f32(bias_bf16)
    return y


def close_to_ref(y_bf16, ref, rtol=1e-2, atol=1e-2):
    """BASELINE gate: |y - bf16(ref)| <= atol + rtol*|bf16(ref)|, elementwise. Returns (ok, worst excess, rel_err)
    where rel_err is the reference harness's gate max|y-ref|/max|ref| (paia-bench/bench/ops/ours_bf16.py:83-89)."""
    y = bf16_bits_to_f32(y_bf16).astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    rb = bf16_bits_to_f32(f32_to_bf16_bits(r.astype(np.float32))).astype(np.float64)
    diff = np.abs(y - rb)
    ok = bool(np.all(diff <= atol + rtol * np.abs(rb)))
    denom = np.abs(r).max() if r.size else 0.0
    rel = float(np.abs(y - r).max() / denom) if denom > 0 else float(np.abs(y).max() if y.size else 0.0)
    excess = float((diff - (atol + rtol * np.abs(rb))).max()) if r.size else 0.0
    return ok, excess, rel
