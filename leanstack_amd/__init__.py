"""leanstack_amd: MI355X (gfx950) BF16 projection path of a Qwen3-4B-shaped decoder.

Hand-written HIP kernels behind a C ABI (include/leanstack_amd.h), a packed
MFMA-tile weight layout, a resident arena planner, and Python entry points
with the names and signatures of leanstack's semantic-runtime dispatch
(src/leanstack/runtime/qwen_explicit.py:963-971).
"""

__version__ = "0.1.0"
