"""Write tests/golden/quant_host_vectors.npz from the REFERENCE's own host-format code.

The reference's src/paia_gemv/quant_host.h is compiled in place by oracle/Makefile into oracle/_ref/libquant_host_ref.so
(see oracle/ref_shim.cpp); this script calls it on seeded inputs and stores inputs + outputs. The fixture pins the
oracle restatement (oracle/paia_oracle.c) wherever the reference checkout is absent (e.g. on the GPU box).

    make -C oracle && python tests/golden/make_golden.py

Contents (all arrays small):
  e4m3_decode      float32[256]   value of every code (NaN for 0x7F/0xFF)           quant_host.h:18-23
  enc_in/enc_out   float32/uint8  e4m3 encode of probe values (random, midpoints, ties, clamps, +-0, NaN) :25-39
  f16_in/f16_out   float32/uint16 fp16 RNE of probe values (subnormals, ties, overflow, NaN)              :41-61
  fp8_W/fp8_q/fp8_scale/fp8_deq     quantize_fp8_rowwise + dequant of a 6x400 matrix with a zero row       :73-85
  i4_W/i4_packed/i4_scales/i4_deq   quantize_int4_g128 + dequant of a 5x512 matrix with a zero group and a
                                    group whose fp16 scale underflows                                       :87-111
"""
import ctypes
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "quant_host_vectors.npz"


def probe_values(rng):
    t = np.array([O.ref_lib().ref_e4m3_decode(c) for c in range(256)], np.float32)
    fin = np.sort(np.unique(np.abs(t[np.isfinite(t)])))
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)           # exact ties between neighbouring codes
    near = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))]).astype(np.float32)
    rand = np.concatenate([rng.uniform(-500, 500, 3000), rng.uniform(-0.02, 0.02, 3000)]).astype(np.float32)
    edge = np.array([0.0, -0.0, 448.0, -448.0, 449.0, 464.0, 480.0, 1e6, -1e6, np.inf, -np.inf, np.nan,
                     2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -6, 1.0, -1.0], np.float32)
    return np.concatenate([mids, -mids, near, rand, edge]).astype(np.float32)


def f16_probe(rng):
    mags = np.exp(rng.uniform(np.log(1e-9), np.log(7e4), 6000)).astype(np.float32)
    signs = np.where(rng.random(6000) < 0.5, -1, 1).astype(np.float32)
    # exact ties halfway between adjacent fp16 values, in the normal and subnormal ranges
    h = np.arange(0, 0x7BFF, 37, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 65536, 1e30, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 0, -0.0, np.inf,
                     np.nan], np.float32)
    return np.concatenate([mags * signs, ties, -ties, edge]).astype(np.float32)


def main():
    R = O.ref_lib()
    if R is None:
        sys.exit("oracle/_ref/libquant_host_ref.so not built (needs the reference checkout; run make -C oracle)")
    rng = np.random.default_rng(20261201)
    dec = np.array([R.ref_e4m3_decode(c) for c in range(256)], np.float32)
    enc_in = probe_values(rng)
    enc_out = np.array([R.ref_e4m3_encode(float(v)) for v in enc_in], np.uint8)
    f16_in = f16_probe(rng)
    f16_out = np.array([R.ref_f32_to_f16_bits(float(v)) for v in f16_in], np.uint16)

    fp8_W = (rng.standard_normal((6, 400)) * 0.02).astype(np.float32)
    fp8_W[2] = 0.0                                                   # amax == 0 -> scale 1
    fp8_W[4, 17] = 3.5                                               # one large outlier
    fp8_q = np.empty(fp8_W.shape, np.uint8)
    fp8_s = np.empty(6, np.float32)
    R.ref_quantize_fp8_rowwise(fp8_W, 6, 400, fp8_q, fp8_s)
    fp8_deq = np.empty(fp8_W.shape, np.float32)
    R.ref_dequant_fp8(fp8_q, fp8_s, 6, 400, fp8_deq)

    i4_W = (rng.standard_normal((5, 512)) * 0.02).astype(np.float32)
    i4_W[1, 128:256] = 0.0                                           # zero group -> scale 1.0, codes 8
    i4_W[3, 256:384] = rng.standard_normal(128).astype(np.float32) * 1e-9   # amax/7 underflows fp16 -> scale 0
    i4_p = np.empty((5, 256), np.uint8)
    i4_s = np.empty((5, 4), np.uint16)
    R.ref_quantize_int4_g128(i4_W, 5, 512, i4_p, i4_s)
    i4_deq = np.empty(i4_W.shape, np.float32)
    R.ref_dequant_int4(i4_p, i4_s, 5, 512, i4_deq)

    np.savez_compressed(OUT, e4m3_decode=dec, enc_in=enc_in, enc_out=enc_out, f16_in=f16_in, f16_out=f16_out,
                        fp8_W=fp8_W, fp8_q=fp8_q, fp8_scale=fp8_s, fp8_deq=fp8_deq,
                        i4_W=i4_W, i4_packed=i4_p, i4_scales=i4_s, i4_deq=i4_deq)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
