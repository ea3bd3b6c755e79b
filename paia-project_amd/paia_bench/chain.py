"""The Llama-3.1-8B decode-step linear chain at M=1, on one GPU, as one HIP graph.

32 layers x (qkv 6144x4096, o 4096x4096, gate_up 28672x4096, down 4096x14336) in one weight format (INT4 g128
asymmetric or FP8 W8A16), then the bf16 lm_head 128256x4096: 129 GEMV launches on one stream, captured into one
graph and replayed. Every layer has its own buffers: layer 0 holds the BASELINE seeded operands (CPU generator,
seed 1000 + N + K), checked against the CPU reference before timing; layers 1..31 are drawn with the same
distributions on the device from a generator seeded 1000 + N + K + 7919. The whole chain (4.68 GB INT4, 8.04 GB FP8)
streams from HBM on every replay; the 256 MiB Infinity Cache holds none of it across a replay.

The launches are serialised exactly as in a decode step, in its order (layer by layer: qkv, o, gate_up, down; one
stream, each GEMV starts when the previous one has finished). The GEMV inputs x are fixed per launch: this chain
measures the linear layers only; attention, norms and activations that would sit between them are not part of the
path.
"""
from __future__ import annotations

import torch

from paia_gemv.shapes import LAYER, LM_HEAD, gemv_bytes

from .cases import GemvCase
from .timing import capture, replay_ms, stats


def build_chain(lib, fmt: str, model: str = "llama31_8b", layers: int = 32, device="cuda", check: bool = True):
    """Returns (launch list, total algorithmic bytes, check results). fmt: 'int4zp' | 'fp8' (| 'bf16' | 'int4')."""
    dev = torch.device(device)
    total = 0
    checks = {}
    cases = []
    for nm, N, K in LAYER[model]:
        case = GemvCase(lib, fmt, N, K, name=f"{fmt}_{nm}_{N}x{K}")
        # copy 0 = the seeded CPU operands of layer 0 (checked), copies 1.. = per-layer device-seeded operands
        case.build(layers, dev, seed=1000 + N + K + 7919)
        if check:
            rows = list(range(0, N, max(1, N // 64)))
            checks[case.name] = case.check(rows=rows)
        cases.append(case)
        total += layers * case.bytes()["total"]
    # decode order: layer 0's qkv, o, gate_up, down, then layer 1's, ...
    launches = [(case, l) for l in range(layers) for case in cases]
    N, K = LM_HEAD[model]
    head = GemvCase(lib, "bf16", N, K, name=f"bf16_lm_head_{N}x{K}")
    head.build(1, dev)
    if check:
        checks[head.name] = head.check(rows=list(range(0, N, N // 64)))
    launches.append((head, 0))
    total += head.bytes()["total"]
    return launches, total, checks


def sample_rows(N: int, n: int = 64) -> list:
    """n rows spread over [0, N), the first and the last included."""
    return sorted(set(range(0, N, max(1, N // n))) | {N - 1})


def check_layers(launches, layers, n_rows: int = 64) -> dict:
    """After a replay: the outputs of the given layers (and of the lm_head) against the CPU fp32 reference built
    from those layers' own device operands, on sampled rows. {case name@layer: check result}."""
    out = {}
    for case, i in launches:
        if i in layers or case.name.startswith("bf16_lm_head"):
            out[f"{case.name}@{i}"] = case.check_copy(i, sample_rows(case.N, n_rows))
    return out


def time_chain(launches, replays: int = 20, warmup: int = 3) -> dict:
    """One graph = one decode step's 129 launches; events around each replay on the launch stream."""
    def step():
        for case, i in launches:
            case.call(i)
    g = capture(step, warm=1)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = replay_ms(g, replays)
    del g
    st = stats(ms)
    return {"us_per_token_step": st["median"] * 1e3, "us_p5": st["p5"] * 1e3, "us_p95": st["p95"] * 1e3,
            "replays": st["n"], "launches": len(launches)}


def run_chain(lib, fmt: str, model: str = "llama31_8b", replays: int = 20, log=print) -> dict:
    launches, total, checks = build_chain(lib, fmt, model)
    bad = {k: v for k, v in checks.items() if not v["ok"]}
    if bad:
        raise RuntimeError(f"decode chain {fmt}: correctness gate failed: {bad}")
    t = time_chain(launches, replays)
    # the outputs the replays left: layers 0, 1 and the last, and the lm_head, against their own operands
    after = check_layers(launches, {0, 1, max(i for _, i in launches)})
    bad = {k: v for k, v in after.items() if not v["ok"]}
    if bad:
        raise RuntimeError(f"decode chain {fmt}: outputs after the graph replays failed the gate: {bad}")
    gbps = total / (t["us_per_token_step"] * 1e-6) / 1e9
    log(f"  chain {fmt}: {t['us_per_token_step']:.1f} us/token-step, {gbps:.0f} GB/s over {total / 1e9:.2f} GB")
    res = {"format": fmt, "model": model, "bytes_per_step": total, "gbps": round(gbps, 1),
           "pct_of_8TBps": round(100 * gbps / 8000.0, 1), **{k: round(v, 2) if isinstance(v, float) else v
                                                             for k, v in t.items()},
           "max_rel_err": max(v["rel_err"] for v in checks.values()),
           "replayed_outputs_checked": sorted(after), "replayed_max_rel_err": max(v["rel_err"] for v in after.values())}
    for case in {c for c, _ in launches}:
        case.free()
    torch.cuda.empty_cache()
    return res


__all__ = ["build_chain", "time_chain", "run_chain", "check_layers", "sample_rows", "gemv_bytes"]
