"""Projection shapes and algorithmic byte counts for the M=1 GEMVs.

Shapes follow paia-bench/configs/shapes.yaml:9-49 (weights are [N_out, K_in]; y = x @ W.T). Byte accounting follows
paia-bench/bench/ops/ours_bf16.py:66-67 and ours_quant.py:92-93,131-132: weights + metadata + x read once + y written
once; the asymmetric INT4 format adds its packed zero points (ceil(G/2) bytes per row) and a bias adds 2N.
"""
from __future__ import annotations

LLAMA31_8B = {
    "q_proj": (4096, 4096), "k_proj": (1024, 4096), "v_proj": (1024, 4096), "o_proj": (4096, 4096),
    "gate_proj": (14336, 4096), "up_proj": (14336, 4096), "down_proj": (4096, 14336),
    "qkv_fused": (6144, 4096), "gate_up_fused": (28672, 4096), "lm_head": (128256, 4096),
}
QWEN25_7B = {
    "q_proj": (3584, 3584), "k_proj": (512, 3584), "v_proj": (512, 3584), "o_proj": (3584, 3584),
    "gate_proj": (18944, 3584), "up_proj": (18944, 3584), "down_proj": (3584, 18944),
    "qkv_fused": (4608, 3584), "gate_up_fused": (37888, 3584), "lm_head": (152064, 3584),
}
MODELS = {"llama31_8b": LLAMA31_8B, "qwen25_7b": QWEN25_7B}

# The reference harness's frozen synthetic sweep (paia-bench/configs/shapes.yaml:51-60): BF16 weight bytes from
# 0.25 MiB to 1 GiB in geometric steps at K = 4096 and K = 14336; and its batch sweep M values (:62-64).
SYNTHETIC = {
    "K4096": (4096, [32, 64, 128, 256, 384, 768, 1536, 2816, 5376, 10112, 19200, 36480, 69120, 131072]),
    "K14336": (14336, [32, 64, 128, 256, 384, 768, 1536, 2944, 5504, 10368, 19712, 37504]),
}
BATCH_M = [1, 2, 4, 8, 16]
N_LAYERS = {"llama31_8b": 32, "qwen25_7b": 28}

# The per-layer linear chain of the BASELINE configs: (name, N, K).
LAYER = {
    "llama31_8b": [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)],
    "qwen25_7b": [("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)],
}
LM_HEAD = {"llama31_8b": (128256, 4096), "qwen25_7b": (152064, 3584)}


def gemv_bytes(fmt: str, N: int, K: int, bias: bool = False, M: int = 1) -> dict:
    """Algorithmic bytes of one GEMV with M activation rows: {weights, metadata, act_in, out, total}.
    fmt: 'bf16' | 'fp8' | 'int4' (reference format: fp16 scales, zero 8) | 'int4zp' (bf16 scales + 4-bit zeros).
    act_in = 2MK and out = 2MN, the reference harness's M accounting (paia-bench/bench/ops/cublas_bf16.py:18-21)."""
    G = K // 128
    if fmt == "bf16":
        w, meta = 2 * N * K, 0
    elif fmt == "fp8":
        w, meta = N * K, 4 * N
    elif fmt == "int4":
        w, meta = N * K // 2, 2 * N * G
    elif fmt == "int4zp":
        w, meta = N * K // 2, 2 * N * G + N * ((G + 1) // 2)
    else:
        raise ValueError(fmt)
    d = {"weights": w, "metadata": meta + (2 * N if bias else 0), "act_in": 2 * M * K, "out": 2 * M * N}
    d["total"] = sum(d.values())
    return d
