"""MI355X calibration: achievable streaming-read bandwidth ("B0") and the per-launch floor of graph launches.

    python -m paia_bench.probe [--out PATH]

  * B0 (large): a 2 GiB nontemporal streaming read, best over two probes and their launch shapes (a grid-stride
    loop, and the GEMV's own load path: raw buffer loads of 1-KiB chunks per wave from a persistent grid, two items
    in flight); the reference's dev B0 method (src/tests/gemv_bf16_check.cu:228-252) on MI355X.
  * B0 at the GEMV sizes: reads of S bytes from distinct slices of a 2 GiB buffer, back to back in one graph (the
    same cold-cache rotation the GEMV timings use), so "us for S bytes" is the floor a GEMV of S bytes can reach.
  * launch floor: back-to-back empty kernels in one graph.

    python -m paia_bench.probe --staged [--out PATH]

  * staged floor: the grid-stride read of each BASELINE GEMV's bytes by blocks that first stage 2K bytes (the GEMV's
    x) into LDS behind a barrier, as every GEMV block must before its first item; best over 2-16 blocks per CU, timed
    as the GEMVs are. Beside the read floor it separates what staging x costs any kernel of that shape from what the
    GEMV's own walk costs.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent.parent


def load_probe():
    lib = ctypes.CDLL(str(PKG / "build" / "libpaia_probe.so"))
    lib.paia_probe_read.restype = ctypes.c_int
    lib.paia_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    lib.paia_probe_stream.restype = ctypes.c_int
    lib.paia_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p]
    lib.paia_probe_stream_lead.restype = ctypes.c_int
    lib.paia_probe_stream_lead.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p]
    lib.paia_probe_set_output.restype = ctypes.c_int
    lib.paia_probe_set_output.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.paia_probe_copy.restype = ctypes.c_int
    lib.paia_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    lib.paia_probe_read_staged.restype = ctypes.c_int
    lib.paia_probe_read_staged.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.paia_probe_empty.restype = ctypes.c_int
    lib.paia_probe_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
    return lib


# Launch shapes of the two probes. ("gs", blocks per CU, unroll): the grid-stride loop of 256-thread blocks.
# ("st", U, W, blocks per CU): the GEMV's load path (U 1-KiB chunks per item, W waves per block); at most 32 waves
# per CU, as the GEMV's launches. ("lw", U, blocks per CU): the load path in 8-wave blocks of which only wave 0
# streams, the walk of a split-K GEMV whose rows are one segment long (the BF16 lm_heads at R = 2, U = 8: wave 0 of
# each block streams 14-16 KiB row pairs, consecutive pairs on consecutive blocks); on MI355X, 2 such blocks per CU
# read 1.05 GB faster than any "st" or "gs" shape.
GS_CONFIGS = [("gs", m, u) for m in (4, 8, 16) for u in (1, 4)]
LEAD_CONFIGS = [("lw", U, b) for U in (8, 16) for b in (1, 2, 4)]
ST_CONFIGS = [("st", U, W, b) for U in (1, 2, 4, 8, 16) for W, b in ((4, 2), (4, 4), (4, 8), (8, 1), (8, 2), (8, 4),
                                                                      (16, 1), (16, 2)) if U < 16 or W < 16]
PROBE_CONFIGS = GS_CONFIGS + ST_CONFIGS + LEAD_CONFIGS
# the read floor at a GEMV's byte count sweeps a subset (every grid-stride shape, the GEMV-path probe at every item
# size on the four launch shapes the GEMVs use most, and the lead-wave walk)
SIZED_CONFIGS = GS_CONFIGS + [("st", U, W, b) for U in (1, 2, 4, 8, 16) for W, b in ((4, 8), (8, 2), (8, 4), (16, 1))
                              if U < 16 or W < 16] + LEAD_CONFIGS


def probe_launch(P, cfg, ptr, nbytes, sink_ptr, cus, stream):
    """One read of nbytes at ptr with launch shape cfg (an entry of PROBE_CONFIGS)."""
    if cfg[0] == "gs":
        rc = P.paia_probe_read(ptr, nbytes, sink_ptr, cus * cfg[1], cfg[2], stream)
    elif cfg[0] == "lw":
        rc = P.paia_probe_stream_lead(ptr, nbytes, sink_ptr, cfg[1], cus * cfg[2], stream)
    else:
        rc = P.paia_probe_stream(ptr, nbytes, sink_ptr, cfg[1], cfg[2], cus * cfg[3], stream)
    if rc:
        raise RuntimeError(f"probe {cfg} rc {rc}")


# The screen of every launch shape times a few replays straight after capture; the FINALISTS best shapes are then
# timed the way one allocation of a GEMV is (paia_bench.timing.time_per_call_us: the same rotation, >= 200 ms and 20
# calls of warm-up, then 200 ms of samples, 30 at least; the median), so a floor and a GEMV time come from the same
# clock state and the same statistic.
FINALISTS = 3


def _final_us(P, cfg, S, slices, sink, cus):
    """µs per read of S bytes with launch shape cfg, rotating over the slice pointers, timed as the GEMVs are."""
    from paia_gemv.loader import current_raw_stream

    from .timing import time_per_call_us
    n = len(slices)
    return time_per_call_us(lambda i: probe_launch(P, cfg, slices[i % n], S, sink.data_ptr(), cus,
                                                   current_raw_stream()), n)["us"]


def b0_large(P, buf, sink, cus, configs=PROBE_CONFIGS, log=print):
    """B0: the best streaming-read rate (GB/s) over the probes' launch shapes, reading all of `buf` (< 2 GiB): a
    screen of every shape (three reads per graph replay, median of 5 replays), then the FINALISTS best timed as the
    GEMVs are. Returns (GB/s, best config)."""
    from paia_gemv.loader import current_raw_stream

    from .timing import capture, replay_ms, stats
    total = buf.numel()
    screen = []
    for cfg in configs:
        g = capture(lambda: [probe_launch(P, cfg, buf.data_ptr(), total, sink.data_ptr(), cus, current_raw_stream())
                             for _ in range(3)], warm=1)
        ms = stats(replay_ms(g, 5))["median"] / 3
        del g
        log(f"[b0] {cfg}: {total / (ms * 1e-3) / 1e9:.0f} GB/s (screen)")
        screen.append((ms, cfg))
    best = (0.0, None)
    for _, cfg in sorted(screen)[:FINALISTS]:
        gbps = total / (_final_us(P, cfg, total, [buf.data_ptr()], sink, cus) * 1e-6) / 1e9
        log(f"[b0] {cfg}: {gbps:.0f} GB/s")
        if gbps > best[0]:
            best = (gbps, cfg)
    return best


def slice_plan(buf_bytes: int, S: int) -> tuple:
    """(slice stride, number of slices) for reads of S bytes rotating over a buffer of buf_bytes: slices start every
    stride bytes (S rounded up to 256) and every slice lies wholly inside the buffer. One slice when only one fits
    (such a read is several times the 256 MiB last-level cache, so it cannot be served from it anyway)."""
    if S <= 0 or S > buf_bytes:
        raise ValueError(f"read of {S} bytes does not fit the {buf_bytes}-byte probe buffer")
    stride = (S + 255) // 256 * 256
    n = max(1, (buf_bytes - S) // stride + 1)
    assert (n - 1) * stride + S <= buf_bytes
    return stride, n


def b0_sized(P, buf, sink, cus, S: int, configs=SIZED_CONFIGS, y=None, nout: int = 0) -> dict:
    """The read floor for S bytes: reads of S bytes from distinct slices of `buf`, back to back in one graph (the
    GEMV timings' cold-cache rotation); a screen of every launch shape, then the best µs per read of the FINALISTS
    timed as the GEMVs are. With nout > 0 (y: a device tensor of at least nout bf16), also the I/O floor: reads of S
    bytes that also write nout bf16 outputs, the best of the read finalists and the two best grid-stride shapes of the
    screen (whose writes come at the very end), timed the same way (io_us, io_cfg)."""
    from paia_gemv.loader import current_raw_stream

    from .timing import capture, replay_ms, stats
    S16, n = slice_plan(buf.numel(), S)
    slices = [buf.data_ptr() + j * S16 for j in range(n)]
    R = min(2000, max(50, int(5e-3 / (S / 6e12))))
    screen = []
    for cfg in configs:
        g = capture(lambda: [probe_launch(P, cfg, slices[j % n], S, sink.data_ptr(), cus, current_raw_stream())
                             for j in range(R)], warm=1)
        screen.append((stats(replay_ms(g, 3))["median"] * 1e3 / R, cfg))
        del g
    finalists = [cfg for _, cfg in sorted(screen)[:FINALISTS]]
    best = min((_final_us(P, cfg, S, slices, sink, cus), cfg) for cfg in finalists)
    out = {"bytes": S, "us": best[0], "gbps": S / (best[0] * 1e-6) / 1e9, "cfg": list(best[1])}
    if nout > 0:
        if y is None or y.numel() * y.element_size() < 2 * nout:
            raise ValueError("the I/O floor needs an output buffer of nout bf16")
        if P.paia_probe_set_output(y.data_ptr(), nout):
            raise RuntimeError(f"probe output of {nout} values refused")
        gs_best = [cfg for _, cfg in sorted(screen) if cfg[0] == "gs"][:2]
        try:
            io = min((_final_us(P, cfg, S, slices, sink, cus), cfg) for cfg in dict.fromkeys(finalists + gs_best))
        finally:
            P.paia_probe_set_output(None, 0)
        out.update(io_us=io[0], io_cfg=list(io[1]), nout=nout)
    return out


STAGED_BLOCKS_PER_CU = (2, 4, 8, 16)


def staged_floor(P, buf, sink, x, cus, S: int, xbytes: int) -> dict:
    """µs per read of S bytes whose blocks first stage xbytes of x into LDS (paia_probe_read_staged), over the slices
    of `buf` as b0_sized rotates them, best over STAGED_BLOCKS_PER_CU, timed as the GEMVs are."""
    from paia_gemv.loader import current_raw_stream

    from .timing import time_per_call_us
    S16, n = slice_plan(buf.numel(), S)
    slices = [buf.data_ptr() + j * S16 for j in range(n)]
    best = None
    for b in STAGED_BLOCKS_PER_CU:
        def call(i, b=b):
            rc = P.paia_probe_read_staged(slices[i % n], S, sink.data_ptr(), cus * b, x.data_ptr(), xbytes,
                                          current_raw_stream())
            if rc:
                raise RuntimeError(f"staged probe rc {rc}")
        us = time_per_call_us(call, n)["us"]
        if best is None or us < best[0]:
            best = (us, b)
    return {"bytes": S, "x_bytes": xbytes, "us": best[0], "blocks_per_cu": best[1]}


def main_staged(out=None) -> int:
    import torch

    from paia_gemv.shapes import LAYER, gemv_bytes
    P = load_probe()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    buf = torch.empty(2 * 2 ** 30 - 2 ** 20, dtype=torch.uint8, device=dev)
    buf.random_(0, 255)
    x = torch.empty(65536, dtype=torch.uint8, device=dev)
    x.random_(0, 255)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    res = {"cus": cus, "staged": {}}
    for fmt in ("bf16", "fp8", "int4zp"):
        for nm, N, K in LAYER["llama31_8b"] + LAYER["qwen25_7b"]:
            if 2 * K > 65536:
                continue
            key = f"{fmt}_{N}x{K}"
            r = staged_floor(P, buf, sink, x, cus, gemv_bytes(fmt, N, K)["total"], 2 * K)
            res["staged"][key] = r
            print(f"[staged] {key:22s} {r['bytes'] / 2**20:8.2f} MiB  x {r['x_bytes']:6d} B  {r['us']:7.2f} us "
                  f"({r['blocks_per_cu']} blocks/CU)", flush=True)
    if out:
        Path(out).parent.mkdir(parents=True, exist_ok=True)
        Path(out).write_text(json.dumps(res, indent=1))
    return 0


def main(argv=None):
    import torch

    from paia_gemv.loader import current_raw_stream
    from paia_gemv.shapes import LAYER, gemv_bytes

    from .timing import HBM_PEAK_GBPS, capture, replay_ms, stats

    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=None)
    ap.add_argument("--staged", action="store_true", help="only the staged floors of the BASELINE GEMVs")
    a = ap.parse_args(argv)
    if a.staged:
        return main_staged(a.out)
    P = load_probe()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    total = 2 * 2 ** 30 - 2 ** 20       # < 2 GiB: the GEMV-path probe's limit per launch
    buf = torch.empty(total, dtype=torch.uint8, device=dev)
    buf.random_(0, 255)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    res = {"cus": cus}

    # B0 large
    best = b0_large(P, buf, sink, cus, log=lambda m: print(m, flush=True))
    res["b0_gbps"] = best[0]
    res["b0_cfg"] = list(best[1])
    print(f"[b0] best {best[0]:.0f} GB/s ({100 * best[0] / HBM_PEAK_GBPS:.1f}% of 8 TB/s) at {best[1]}", flush=True)

    # B0 at the GEMV sizes
    sizes = {}
    for fmt in ("bf16", "fp8", "int4zp"):
        for nm, N, K in LAYER["llama31_8b"] + LAYER["qwen25_7b"]:
            sizes[f"{fmt}_{N}x{K}"] = gemv_bytes(fmt, N, K)["total"]
    res["sized"] = {}
    for key, S in sorted(sizes.items(), key=lambda kv: kv[1]):
        r = b0_sized(P, buf, sink, cus, S)
        res["sized"][key] = r
        print(f"[b0 sized] {key:22s} {S / 2**20:8.2f} MiB  {r['us']:7.2f} us  {r['gbps']:6.0f} GB/s", flush=True)

    # launch floor
    for grid in (1, 256, 2048):
        g = capture(lambda: [P.paia_probe_empty(grid, current_raw_stream()) for _ in range(1000)], warm=1)
        us = stats(replay_ms(g, 5))["median"] * 1e3 / 1000
        del g
        res[f"empty_launch_us_grid{grid}"] = us
        print(f"[launch] empty kernel grid {grid}: {us:.2f} us per launch in a graph", flush=True)
    if a.out:
        Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.out).write_text(json.dumps(res, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
