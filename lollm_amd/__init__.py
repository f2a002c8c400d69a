"""lollm_amd -- the qwen3_5 MTP speculative-decode step on MI355X (gfx950).

Python host code on PyTorch-ROCm calling hand-written HIP kernels through the C ABI
declared in include/lollm_amd.h (library: lollm_amd/_native/liblollm_amd.so, built by
`python -m lollm_amd.build`).  There is no CPU or fallback path.
"""

__all__ = ["ops", "qwen3_5"]
