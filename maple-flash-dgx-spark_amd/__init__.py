"""maple_amd: MI355X-native (gfx950) packed-ternary MoE decode path.

A drop-in for the hot path of maple-run: the packed ternary GEMV, the fused MoE
router, expert dispatch, the ternary expert kernels (SwiGLU, down projection,
top-k combine), the 4-bit RTN lm_head and the norms around them.  Every kernel
is hand-written HIP behind the C ABI in ``include/maple_amd.h``; this package
is the host-side mirror of the reference's Python interface
(``src/maple_run/kernels/__init__.py``, ``src/maple_run/linear.py``).

The directory name is not a Python identifier, so it is imported under the
name ``maple_amd`` (see ``load_package`` in ``__graft_entry__.py``).
"""

from __future__ import annotations

__all__ = ["kernels", "linear", "moe", "model", "synthetic"]
