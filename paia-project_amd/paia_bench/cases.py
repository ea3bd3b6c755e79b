"""One GEMV configuration on the device: n_copies operand sets for cache-defeating rotation and a launch closure.

Copy 0 holds the seeded BASELINE operands (paia_bench.inputs), the one checked for correctness before any timing
(as paia-bench/bench/run.py:236-240 gates cells). Copies 1.. are drawn on the device with the same distributions
(the reference fills them with random codes, paia-bench/bench/ops/ours_quant.py:3-6; the kernels have no
data-dependent control flow, so timing does not depend on the values either way).
"""
from __future__ import annotations

import torch

from paia_gemv import quant
from paia_gemv.shapes import gemv_bytes

from .inputs import make_operands, to_device

REF_ROWS = 8192     # rows per chunk of the fp32 reference (paia-bench/bench/ops/cublas_bf16.py:11)

# Every M = 1 GEMV of the BASELINE configs: (config, format, model, projection, N, K, bias). configs[0] BF16 o_proj,
# configs[1] the four FP8 Llama-3.1-8B shapes, configs[2] the four INT4 (asymmetric g128) Llama shapes, configs[3] the
# Qwen2.5-7B shapes in all three formats (qkv with its bias) and the bf16 lm_head, configs[4]'s bf16 Llama lm_head.
LLAMA_LAYER = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]
QWEN_LAYER = [("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)]
BASELINE_GEMVS = ([("configs[1]", "fp8", "llama", nm, N, K, False) for nm, N, K in LLAMA_LAYER]
                  + [("configs[0]", "bf16", "llama", "o", 4096, 4096, False)]
                  + [("configs[2]", "int4zp", "llama", nm, N, K, False) for nm, N, K in LLAMA_LAYER]
                  + [("configs[3]", f, "qwen", nm, N, K, nm == "qkv") for f in ("bf16", "fp8", "int4zp")
                     for nm, N, K in QWEN_LAYER]
                  + [("configs[3]", "bf16", "qwen", "lm_head", 152064, 3584, False),
                     ("configs[4]", "bf16", "llama", "lm_head", 128256, 4096, False)])


def case_name(fmt, model, nm, N, K, bias) -> str:
    """The name a BASELINE GEMV goes by in bench.py's record and the counter summaries."""
    return f"{fmt}_{model}_{nm}{'_bias' if bias else ''}_{N}x{K}"


def kernel_name(lib, fmt, variant, N, K) -> str:
    """The template instance a call launches (as rocprofv3 names it): gemv_kernel, or gemv_kernel43 for INT4 launches
    with few weight loads per wave (either with the suffix _dr when no wave takes more than two items), with the
    variant's knobs; gemv_kernel_xg (its fixed knobs) for K beyond the LDS."""
    fam = {"bf16": lib.variants, "fp8": lib.variants_fp8}.get(fmt, lib.variants_int4)
    v = fam[variant]
    F = {"bf16": 0, "fp8": 1, "int4": 2, "int4zp": 3}[fmt]
    aux = (2 if v["S"] else 0) if fmt == "bf16" else 2
    k = lib.launch_kind(fmt, N, K, variant)
    if k == "gemv_kernel_xg":
        return f"paia::gemv_kernel_xg<{F}, 1, 2, 8, {aux}, true>"
    return f"paia::{k}<{F}, {v['R']}, {v['U']}, {v['W']}, {aux}, {'true' if v['H'] else 'false'}>"


def kind_of(fmt: str) -> str:
    return "int4" if fmt.startswith("int4") else fmt


class GemvCase:
    """mode: 'fused' (the M = 1 kernels), 'naive' / 'unfused' (INT4 controls), or 'batch' (the small-batch matrix-core
    kernels, M = 1..16 activation rows; `variant` then indexes lib.variants_batch[fmt])."""

    def __init__(self, lib, fmt: str, N: int, K: int, bias: bool = False, variant: int | None = None,
                 mode: str = "fused", name: str | None = None, M: int = 1):
        self.lib, self.fmt, self.N, self.K, self.bias, self.mode, self.M = lib, fmt, N, K, bias, mode, M
        assert M == 1 or mode == "batch", "M > 1 runs the batch kernels"
        self.name = name or (f"{fmt}_{N}x{K}" if mode != "batch" else f"{fmt}_M{M}_{N}x{K}")
        if variant is not None:
            self.variant = int(variant)
        elif mode == "batch":
            self.variant = lib.batch_pick_variant(fmt, M, N, K)
        else:
            self.variant = lib.pick_variant(fmt, N, K)
        self.copies: list = []
        self.ptrs: list = []
        self.scratch = None
        self.ops0 = None

    # ---- accounting --------------------------------------------------------------------------------------
    def bytes(self) -> dict:
        return gemv_bytes(self.fmt, self.N, self.K, self.bias, self.M)

    def footprint(self) -> int:
        return self.bytes()["total"]

    # ---- operands ----------------------------------------------------------------------------------------
    def _random_copy(self, dev, g):
        """Another operand set with the BASELINE distributions (paia_bench.inputs), drawn on the device."""
        N, K, G = self.N, self.K, self.K // 128
        c = {"N": N, "K": K}
        if self.fmt == "bf16":
            c["W"] = (0.02 * torch.randn(N, K, device=dev, generator=g)).to(torch.bfloat16)
        elif self.fmt == "fp8":
            c["Wq"], c["scale"] = quant.quantize_fp8_rowwise(0.02 * torch.randn(N, K, device=dev, generator=g))
        elif self.fmt == "int4":
            c["Wq"], c["scales"] = quant.quantize_int4_g128(0.02 * torch.randn(N, K, device=dev, generator=g))
        else:
            c["Wq"] = torch.randint(0, 256, (N, K // 2), device=dev, generator=g, dtype=torch.uint8)
            c["scales"] = (0.001 + 0.009 * torch.rand(N, G, device=dev, generator=g)).to(torch.bfloat16)
            c["zeros"] = quant.pack_zeros(torch.randint(0, 16, (N, G), device=dev, generator=g, dtype=torch.uint8))
        c["x"] = torch.randn(*self._xshape(), device=dev, generator=g).to(torch.bfloat16)
        c["bias"] = (0.02 * torch.randn(N, device=dev, generator=g)).to(torch.bfloat16) if self.bias else None
        return c

    def _xshape(self):
        return (self.M, self.K) if self.mode == "batch" else (self.K,)

    def build(self, n_copies: int, device="cuda", seed: int = 1234, host_copy0: bool = True):
        """n_copies operand sets on the device. host_copy0: copy 0 = the seeded CPU operands (make_operands, the
        ones `check` gates); otherwise every copy is drawn on the device (large shapes whose CPU generation would
        dominate a benchmark run; gate copy 0 with check_copy, which builds its reference from device operands)."""
        dev = torch.device(device)
        if not host_copy0:
            assert self.mode != "batch", "device-only operands: M = 1 cases"
            g = torch.Generator(device=dev).manual_seed(seed)
            self.ops0 = None
            self.copies = [self._random_copy(dev, g) for _ in range(n_copies)]
            for c in self.copies:
                c["y"] = torch.empty(self.N, dtype=torch.bfloat16, device=dev)
            if self.mode == "unfused":
                self.scratch = torch.empty(self.N * self.K, dtype=torch.bfloat16, device=dev)
            self.ptrs = [self._ptrs(c) for c in self.copies]
            return self
        self.ops0 = make_operands(self.fmt, self.N, self.K, bias=self.bias)
        if self.mode == "batch":
            # M activation rows: row 0 is the seeded x of make_operands, the others seeded after it
            gx = torch.Generator().manual_seed(2000 + self.M + self.N + self.K)
            xs = torch.randn(self.M, self.K, generator=gx).to(torch.bfloat16)
            xs[0] = self.ops0["x"]
            self.ops0["x"] = xs
        g = torch.Generator(device=dev).manual_seed(seed)
        self.copies = [to_device(self.ops0, dev)] + [self._random_copy(dev, g) for _ in range(n_copies - 1)]
        yshape = (self.M, self.N) if self.mode == "batch" else (self.N,)
        for c in self.copies:
            c["y"] = torch.empty(*yshape, dtype=torch.bfloat16, device=dev)
        if self.mode == "unfused":
            self.scratch = torch.empty(self.N * self.K, dtype=torch.bfloat16, device=dev)
        self.ptrs = [self._ptrs(c) for c in self.copies]
        return self

    @staticmethod
    def _ptr(t):
        return None if t is None else t.data_ptr()

    def _ptrs(self, c):
        p = self._ptr
        if self.fmt == "bf16":
            return (p(c["W"]), p(c["x"]), p(c["bias"]), p(c["y"]))
        if self.fmt == "fp8":
            return (p(c["Wq"]), p(c["scale"]), p(c["x"]), p(c["bias"]), p(c["y"]))
        if self.fmt == "int4":
            return (p(c["Wq"]), p(c["scales"]), p(c["x"]), p(c["y"]))
        return (p(c["Wq"]), p(c["scales"]), p(c["zeros"]), p(c["x"]), p(c["bias"]), p(c["y"]))

    # ---- launch ------------------------------------------------------------------------------------------
    def call(self, i: int, stream=None):
        L, N, K, v = self.lib, self.N, self.K, self.variant
        P = self.ptrs[i]
        if self.mode == "batch":
            M = self.M
            if self.fmt == "bf16":
                W, x, b, y = P
                L.batch_bf16(W, x, b, y, M, N, K, v, stream)
            elif self.fmt == "fp8":
                Wq, s, x, b, y = P
                L.batch_fp8(Wq, s, x, b, y, M, N, K, v, stream)
            elif self.fmt == "int4":
                Wq, s, x, y = P
                L.batch_int4(Wq, s, x, y, M, N, K, v, stream)
            else:
                Wq, s, z, x, b, y = P
                L.batch_int4_zp(Wq, s, z, x, b, y, M, N, K, v, stream)
            return self.copies[i]["y"]
        if self.fmt == "bf16":
            W, x, b, y = P
            if b is None:
                L.bf16(W, x, y, N, K, v, stream)
            else:
                L.bf16_bias(W, x, b, y, N, K, v, stream)
        elif self.fmt == "fp8":
            Wq, s, x, b, y = P
            if b is None:
                L.fp8(Wq, s, x, y, N, K, v, stream)
            else:
                L.fp8_bias(Wq, s, x, b, y, N, K, v, stream)
        elif self.fmt == "int4":
            Wq, s, x, y = P
            if self.mode == "fused":
                L.int4(Wq, s, x, y, N, K, v, stream)
            elif self.mode == "naive":
                L.int4_naive(Wq, s, x, y, N, K, stream)
            else:
                L.int4_unfused(Wq, s, x, y, self.scratch.data_ptr(), N, K, stream)
        else:
            Wq, s, z, x, b, y = P
            L.int4_zp(Wq, s, z, x, b, y, N, K, v, stream)
        return self.copies[i]["y"]

    # ---- correctness gate on copy 0 ----------------------------------------------------------------------
    def reference(self, rows=None) -> torch.Tensor:
        """fp32 reference of copy 0 on the CPU, the reference harness's own method: dequantise with the package's
        torch format definitions (paia_gemv.quant), then x.float() @ Wdeq.t() in chunks of REF_ROWS rows
        (paia-bench/bench/ops/ours_quant.py:69-71, cublas_bf16.py:11,33-38)."""
        o = self.ops0
        idx = torch.arange(self.N) if rows is None else torch.as_tensor(rows, dtype=torch.long)
        x = o["x"].float()
        if x.dim() == 2:                      # batch: one reference row per activation row
            return torch.stack([self._reference_row(x[m], idx) for m in range(x.shape[0])])
        return self._reference_row(x, idx)

    def _reference_row(self, x, idx, weights_bf16: bool = False) -> torch.Tensor:
        o = self.ops0
        out = torch.empty(len(idx), dtype=torch.float32)
        for a in range(0, len(idx), REF_ROWS):
            r = idx[a:a + REF_ROWS]
            if self.fmt == "bf16":
                Wd = o["W"][r].float()
            elif self.fmt == "fp8":
                Wd = quant.dequant_fp8(o["Wq"][r], o["scale"][r])
            elif self.fmt == "int4":
                Wd = quant.dequant_int4(o["Wq"][r], o["scales"][r])
            else:
                Wd = quant.dequant_int4_zp(o["Wq"][r], o["scales"][r], o["zeros"][r])
            if weights_bf16:
                Wd = Wd.to(torch.bfloat16).float()
            out[a:a + len(r)] = Wd @ x
        if o.get("bias") is not None:
            out += o["bias"][idx].float()
        return out

    def check(self, rows=None, rtol=1e-2, atol=1e-2) -> dict:
        """Copy 0 against the CPU reference (all rows, or `rows`): the BASELINE gate (|y - bf16(ref)| <= atol +
        rtol |bf16(ref)|) and the reference harness gate (max|y - ref| / max|ref| < 2e-2, ours_bf16.py:83-89,
        ours_quant.py:73-77)."""
        y = self.call(0)
        torch.cuda.synchronize()
        y = y.cpu().float()
        if rows is not None:
            y = y[..., torch.as_tensor(rows, dtype=torch.long)]
        ref = self.reference(rows)
        if self.mode == "unfused":
            # the unfused control computes with bf16_rn(deq) weights by definition (gemv_int4.cuh:155-174): the
            # element-wise gate compares it with that definition; the harness gate below uses the exact dequant
            idx = torch.arange(self.N) if rows is None else torch.as_tensor(rows, dtype=torch.long)
            refb = self._reference_row(self.ops0["x"].float(), idx, weights_bf16=True).to(torch.bfloat16).float()
        else:
            refb = ref.to(torch.bfloat16).float()
        excess = ((y - refb).abs() - (atol + rtol * refb.abs())).max().item()
        rel = ((y - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        ok = bool(torch.isfinite(y).all().item()) and excess <= 0 and rel < 2e-2
        return {"ok": ok, "rel_err": rel, "worst_excess": excess, "rows_checked": int(len(y))}

    def copy_rows(self, i: int, rows) -> dict:
        """The operands of copy i restricted to `rows` (M = 1 cases), as CPU torch tensors: what a CPU reference of
        those output rows needs. Copies 1.. live only on the device, so this is how their outputs are checked."""
        c = self.copies[i]
        idx = torch.as_tensor(rows, dtype=torch.long, device=c["x"].device)
        out = {"fmt": self.fmt, "N": len(rows), "K": self.K, "x": c["x"].cpu()}
        for k in ("W", "Wq", "scale", "scales", "zeros", "bias"):
            if c.get(k) is not None:
                out[k] = c[k].index_select(0, idx).cpu()
        return out

    def reference_copy(self, i: int, rows) -> torch.Tensor:
        """fp32 CPU reference of copy i's output rows (the harness method of `reference`, on that copy's operands)."""
        o = self.copy_rows(i, rows)
        if self.fmt == "bf16":
            Wd = o["W"].float()
        elif self.fmt == "fp8":
            Wd = quant.dequant_fp8(o["Wq"], o["scale"])
        elif self.fmt == "int4":
            Wd = quant.dequant_int4(o["Wq"], o["scales"])
        else:
            Wd = quant.dequant_int4_zp(o["Wq"], o["scales"], o["zeros"])
        ref = Wd @ o["x"].float()
        if o.get("bias") is not None:
            ref += o["bias"].float()
        return ref

    def check_copy(self, i: int, rows, rtol=1e-2, atol=1e-2) -> dict:
        """Copy i's output as it stands (no launch: e.g. after a graph replay) against reference_copy, with the
        gates of `check`."""
        torch.cuda.synchronize()
        y = self.copies[i]["y"].cpu().float()[torch.as_tensor(rows, dtype=torch.long)]
        ref = self.reference_copy(i, rows)
        refb = ref.to(torch.bfloat16).float()
        excess = ((y - refb).abs() - (atol + rtol * refb.abs())).max().item()
        rel = ((y - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        ok = bool(torch.isfinite(y).all().item()) and excess <= 0 and rel < 2e-2
        return {"ok": ok, "rel_err": rel, "worst_excess": excess, "rows_checked": int(len(y))}

    def free(self):
        self.copies, self.ptrs, self.scratch = [], [], None
