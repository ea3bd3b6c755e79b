"""paia_gemv for MI355X (gfx950): fused M=1 GEMV in BF16, FP8 W8A16 and INT4 W4A16 g128.

Same package surface as the reference's src/paia_gemv/__init__.py (`GemvLib`, `load_lib`, `quant`), plus
`ops` (torch.library custom ops) and `shapes` (the Llama-3.1-8B / Qwen2.5-7B projection shapes).
"""
from .loader import GemvLib, load_lib  # noqa: F401
