"""ctypes loader for libpaia_gemv.so, the gfx950 HIP build (no torch ABI dependency in the library itself).

Drop-in for src/paia_gemv/loader.py:12-109: same `find_lib`, `current_raw_stream`, `GemvLib` (attributes `path`,
`n_variants`, `variants`, `variants_fp8`, `variants_int4`; methods `bf16`, `fp8`, `int4`, `int4_naive`,
`int4_unfused`) and `load_lib`. Pointers are plain ints; a nonzero return code raises RuntimeError. Launches go on
torch's current stream, so calls can be captured into a HIP graph (torch.cuda.CUDAGraph on ROCm).

Additions for the gfx950 build: `bf16_bias`, `fp8_bias`, `int4_zp` (asymmetric INT4 with optional bias),
`dequant_fp8`, `dequant_int4`, `dequant_int4_zp`, `quantize_fp8_rowwise`, `quantize_int4_g128`,
`quantize_int4_zp_g128`, `pick_variant`, `launch_kind`, `build_info`.
"""
from __future__ import annotations

import ctypes
import os
import platform
from pathlib import Path

_PKG_ROOT = Path(__file__).resolve().parent.parent       # paia-project_amd/


def find_lib() -> str:
    """PAIA_GEMV_LIB, else <pkg>/build/<machine>/libpaia_gemv.so, else <pkg>/build/libpaia_gemv.so."""
    env = os.environ.get("PAIA_GEMV_LIB")
    cands = [env] if env else []
    cands += [str(_PKG_ROOT / "build" / platform.machine() / "libpaia_gemv.so"),
              str(_PKG_ROOT / "build" / "libpaia_gemv.so")]
    for c in cands:
        if c and os.path.exists(c):
            return c
    raise FileNotFoundError("libpaia_gemv.so not found (run `python paia-project_amd/build.py`, or set "
                            "PAIA_GEMV_LIB). Tried: " + ", ".join(c for c in cands if c))


def current_raw_stream():
    import torch
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device())


_P = ctypes.c_void_p
_I = ctypes.c_int
KINDS = {"bf16": 0, "fp8": 1, "int4": 2, "int4zp": 3}


class GemvLib:
    CODES = "-1: no such variant; -2: shape or alignment outside the contract; > 0: HIP error"

    def __init__(self, path=None):
        self.path = path or find_lib()
        lib = ctypes.CDLL(self.path)
        sig = {
            "paia_gemv_bf16": [_P, _P, _P, _I, _I, _I, _P],
            "paia_gemv_bf16_bias": [_P, _P, _P, _P, _I, _I, _I, _P],
            "paia_gemv_fp8": [_P, _P, _P, _P, _I, _I, _I, _P],
            "paia_gemv_fp8_bias": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
            "paia_gemv_int4": [_P, _P, _P, _P, _I, _I, _I, _P],
            "paia_gemv_int4_naive": [_P, _P, _P, _P, _I, _I, _P],
            "paia_gemv_int4_unfused": [_P, _P, _P, _P, _P, _I, _I, _P],
            "paia_gemv_int4_unfused_noalloc": [_P, _P, _P, _P, _I, _I, _P],
            "paia_gemv_int4_zp": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
            "paia_dequant_fp8": [_P, _P, _P, _I, _I, _P],
            "paia_dequant_int4": [_P, _P, _P, _I, _I, _P],
            "paia_dequant_int4_zp": [_P, _P, _P, _P, _I, _I, _P],
            "paia_quantize_fp8_rowwise": [_P, _P, _P, _I, _I, _P],
            "paia_quantize_int4_g128": [_P, _P, _P, _I, _I, _P],
            "paia_quantize_int4_zp_g128": [_P, _P, _P, _P, _I, _I, _P],
            "paia_gemv_pick_variant": [_I, _I, _I],
            "paia_gemv_launch_kind": [_I, _I, _I, _I],
            "paia_gemv_bf16_variant_count": [],
            "paia_gemv_bf16_variant_info": [_I] + [ctypes.POINTER(_I)] * 5,
            "paia_gemv_batch_variant_count": [_I],
            "paia_gemv_batch_variant_info": [_I, _I] + [ctypes.POINTER(_I)] * 5,
            "paia_gemv_batch_pick_variant": [_I, _I, _I, _I],
            "paia_gemv_batch_bf16": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
            "paia_gemv_batch_fp8": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
            "paia_gemv_batch_int4": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
            "paia_gemv_batch_int4_zp": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
        }
        for name, argtypes in sig.items():
            fn = getattr(lib, name)
            fn.restype = _I
            fn.argtypes = argtypes
        lib.paia_gemv_build_info.restype = ctypes.c_char_p
        lib.paia_gemv_build_info.argtypes = []
        self.variants_fp8 = self._qvariants(lib, "fp8")
        self.variants_int4 = self._qvariants(lib, "int4")
        self._lib = lib
        self._fn = lib.paia_gemv_bf16
        self.n_variants = lib.paia_gemv_bf16_variant_count()
        self.variants = []
        for v in range(self.n_variants):
            R, U, W, S, H = (_I() for _ in range(5))
            assert lib.paia_gemv_bf16_variant_info(v, *map(ctypes.byref, (R, U, W, S, H))) == 0
            self.variants.append({"id": v, "R": R.value, "U": U.value, "W": W.value, "S": S.value, "H": H.value})
        self.variants_batch = {}
        for kind, k in KINDS.items():
            vs = []
            for v in range(lib.paia_gemv_batch_variant_count(k)):
                P, U, W, S, X = (_I() for _ in range(5))
                assert lib.paia_gemv_batch_variant_info(k, v, *map(ctypes.byref, (P, U, W, S, X))) == 0
                vs.append({"id": v, "P": P.value, "U": U.value, "W": W.value, "S": S.value, "X": X.value})
            self.variants_batch[kind] = vs

    @staticmethod
    def _qvariants(lib, kind):
        count = getattr(lib, f"paia_gemv_{kind}_variant_count")
        count.restype = _I
        count.argtypes = []
        info = getattr(lib, f"paia_gemv_{kind}_variant_info")
        info.restype = _I
        info.argtypes = [_I] + [ctypes.POINTER(_I)] * 4
        out = []
        for v in range(count()):
            R, U, W, H = (_I() for _ in range(4))
            assert info(v, *map(ctypes.byref, (R, U, W, H))) == 0
            out.append({"id": v, "R": R.value, "U": U.value, "W": W.value, "S": 0, "H": H.value})
        return out

    @classmethod
    def _check(cls, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} returned {rc} ({cls.CODES})")

    @staticmethod
    def _st(stream):
        return current_raw_stream() if stream is None else stream

    # ---- reference surface -------------------------------------------------------------------------------
    def bf16(self, W_ptr, x_ptr, y_ptr, N, K, variant, stream=None):
        """BF16 weights: the output vector (N bf16 values) from the row-major N x K matrix and the K-vector, each
        passed as a device address (int)."""
        rc = self._fn(W_ptr, x_ptr, y_ptr, N, K, variant, self._st(stream))
        if rc != 0:
            raise RuntimeError(f"paia_gemv_bf16 returned {rc} for N={N} K={K} variant {variant} "
                               "(-1: no such variant; -2: K not a multiple of 8 or a pointer not 16-byte aligned; "
                               "> 0: HIP error)")

    def fp8(self, Wq_ptr, scale_ptr, x_ptr, y_ptr, N, K, variant, stream=None):
        """FP8 weights: one e4m3fn byte per weight (N x K), one fp32 scale per output row; bf16 x and y; K a
        multiple of 16."""
        self._check(self._lib.paia_gemv_fp8(Wq_ptr, scale_ptr, x_ptr, y_ptr, N, K, variant, self._st(stream)),
                    "paia_gemv_fp8")

    def int4(self, Wq_ptr, scales_ptr, x_ptr, y_ptr, N, K, variant, stream=None):
        """INT4 weights, two per byte (N x K/2), zero point 8, one fp16 scale per 128 columns of a row; K a multiple
        of 128. The fused kernel."""
        self._check(self._lib.paia_gemv_int4(Wq_ptr, scales_ptr, x_ptr, y_ptr, N, K, variant, self._st(stream)),
                    "paia_gemv_int4")

    def int4_naive(self, Wq_ptr, scales_ptr, x_ptr, y_ptr, N, K, stream=None):
        self._check(self._lib.paia_gemv_int4_naive(Wq_ptr, scales_ptr, x_ptr, y_ptr, N, K, self._st(stream)),
                    "paia_gemv_int4_naive")

    def int4_unfused(self, Wq_ptr, scales_ptr, x_ptr, y_ptr, scratch_ptr, N, K, stream=None):
        self._check(self._lib.paia_gemv_int4_unfused(Wq_ptr, scales_ptr, x_ptr, y_ptr, scratch_ptr, N, K,
                                                     self._st(stream)), "paia_gemv_int4_unfused")

    # ---- gfx950 additions --------------------------------------------------------------------------------
    def int4_unfused_noalloc(self, Wq_ptr, scales_ptr, x_ptr, y_ptr, N, K, stream=None):
        """The unfused control without a workspace argument: the library's static device scratch (for callers that
        cannot allocate; calls that overlap on one GPU race)."""
        self._check(self._lib.paia_gemv_int4_unfused_noalloc(Wq_ptr, scales_ptr, x_ptr, y_ptr, N, K, self._st(stream)),
                    "paia_gemv_int4_unfused_noalloc")

    def bf16_bias(self, W_ptr, x_ptr, bias_ptr, y_ptr, N, K, variant, stream=None):
        self._check(self._lib.paia_gemv_bf16_bias(W_ptr, x_ptr, bias_ptr, y_ptr, N, K, variant, self._st(stream)),
                    "paia_gemv_bf16_bias")

    def fp8_bias(self, Wq_ptr, scale_ptr, x_ptr, bias_ptr, y_ptr, N, K, variant, stream=None):
        self._check(self._lib.paia_gemv_fp8_bias(Wq_ptr, scale_ptr, x_ptr, bias_ptr, y_ptr, N, K, variant,
                                                 self._st(stream)), "paia_gemv_fp8_bias")

    def int4_zp(self, Wq_ptr, scales_ptr, zeros_ptr, x_ptr, bias_ptr, y_ptr, N, K, variant, stream=None):
        """Asymmetric INT4: scales bf16 [N,G], zeros [N,ceil(G/2)] (2 nibbles/byte), bias bf16 [N] or None."""
        self._check(self._lib.paia_gemv_int4_zp(Wq_ptr, scales_ptr, zeros_ptr, x_ptr, bias_ptr, y_ptr, N, K, variant,
                                                self._st(stream)), "paia_gemv_int4_zp")

    def dequant_fp8(self, Wq_ptr, scale_ptr, out_ptr, N, K, stream=None):
        self._check(self._lib.paia_dequant_fp8(Wq_ptr, scale_ptr, out_ptr, N, K, self._st(stream)), "paia_dequant_fp8")

    def dequant_int4(self, Wq_ptr, scales_ptr, out_ptr, N, K, stream=None):
        self._check(self._lib.paia_dequant_int4(Wq_ptr, scales_ptr, out_ptr, N, K, self._st(stream)),
                    "paia_dequant_int4")

    def dequant_int4_zp(self, Wq_ptr, scales_ptr, zeros_ptr, out_ptr, N, K, stream=None):
        self._check(self._lib.paia_dequant_int4_zp(Wq_ptr, scales_ptr, zeros_ptr, out_ptr, N, K, self._st(stream)),
                    "paia_dequant_int4_zp")

    def quantize_fp8_rowwise(self, W_ptr, q_ptr, scale_ptr, N, K, stream=None):
        """fp32 W [N,K] -> e4m3 q [N,K], fp32 scale [N] on the device (quant.py:8-13 semantics)."""
        self._check(self._lib.paia_quantize_fp8_rowwise(W_ptr, q_ptr, scale_ptr, N, K, self._st(stream)),
                    "paia_quantize_fp8_rowwise")

    def quantize_int4_g128(self, W_ptr, packed_ptr, scales_ptr, N, K, stream=None):
        """fp32 W [N,K] -> packed [N,K/2], fp16 scales [N,K/128] on the device (quant.py:20-31 semantics)."""
        self._check(self._lib.paia_quantize_int4_g128(W_ptr, packed_ptr, scales_ptr, N, K, self._st(stream)),
                    "paia_quantize_int4_g128")

    def quantize_int4_zp_g128(self, W_ptr, packed_ptr, scales_ptr, zeros_ptr, N, K, stream=None):
        """fp32 W [N,K] -> asymmetric INT4: packed [N,K/2], bf16 scales [N,G], zeros [N,ceil(G/2)] on the device."""
        self._check(self._lib.paia_quantize_int4_zp_g128(W_ptr, packed_ptr, scales_ptr, zeros_ptr, N, K,
                                                         self._st(stream)), "paia_quantize_int4_zp_g128")

    def pick_variant(self, kind, N, K):
        """Library's per-shape variant: kind 'bf16' | 'fp8' | 'int4' | 'int4zp' (an index of variants_int4)."""
        return self._lib.paia_gemv_pick_variant(KINDS[kind], N, K)

    # ---- small batch (M = 1..16 activation rows, x [M,K] and y [M,N] bf16 row-major) -------------------------
    KERNELS = ("gemv_kernel", "gemv_kernel43", "gemv_kernel_xg", "gemv_kernel_dr", "gemv_kernel43_dr")

    def launch_kind(self, kind, N, K, variant):
        """The kernel a call of `variant` runs at (N, K), as a profiler names it: "gemv_kernel", "gemv_kernel43" (INT4
        launches with few weight loads per wave) or "gemv_kernel_xg" (K beyond the LDS staging)."""
        k = self._lib.paia_gemv_launch_kind(KINDS[kind], N, K, variant)
        if k < 0:
            raise ValueError(f"paia_gemv_launch_kind({kind}, {N}, {K}, {variant}) returned {k}")
        return self.KERNELS[k]

    def batch_pick_variant(self, kind, M, N, K):
        """The library's default small-batch variant (an index of variants_batch[kind]); -1 if M is out of range."""
        return self._lib.paia_gemv_batch_pick_variant(KINDS[kind], M, N, K)

    def batch_bf16(self, W_ptr, x_ptr, bias_ptr, y_ptr, M, N, K, variant=-1, stream=None):
        self._check(self._lib.paia_gemv_batch_bf16(W_ptr, x_ptr, bias_ptr, y_ptr, M, N, K, variant, self._st(stream)),
                    "paia_gemv_batch_bf16")

    def batch_fp8(self, Wq_ptr, scale_ptr, x_ptr, bias_ptr, y_ptr, M, N, K, variant=-1, stream=None):
        self._check(self._lib.paia_gemv_batch_fp8(Wq_ptr, scale_ptr, x_ptr, bias_ptr, y_ptr, M, N, K, variant,
                                                  self._st(stream)), "paia_gemv_batch_fp8")

    def batch_int4(self, Wq_ptr, scales_ptr, x_ptr, y_ptr, M, N, K, variant=-1, stream=None):
        self._check(self._lib.paia_gemv_batch_int4(Wq_ptr, scales_ptr, x_ptr, y_ptr, M, N, K, variant,
                                                   self._st(stream)), "paia_gemv_batch_int4")

    def batch_int4_zp(self, Wq_ptr, scales_ptr, zeros_ptr, x_ptr, bias_ptr, y_ptr, M, N, K, variant=-1, stream=None):
        self._check(self._lib.paia_gemv_batch_int4_zp(Wq_ptr, scales_ptr, zeros_ptr, x_ptr, bias_ptr, y_ptr, M, N, K,
                                                      variant, self._st(stream)), "paia_gemv_batch_int4_zp")

    def build_info(self):
        return self._lib.paia_gemv_build_info().decode()


_lib = None


def load_lib():
    global _lib
    if _lib is None:
        _lib = GemvLib()
    return _lib
