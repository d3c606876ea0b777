"""qwfnfer_amd -- MI355X (gfx950) q8_0 KV cache and Qwen Sparse Attention decode path.

The kernels and the C ABI live in ``libqwfn_qsa.so`` (built from ``csrc/`` by
``qwfnfer_amd.build``); ``qwfnfer_amd.qsa`` is the host-side mirror of the
reference engine's cache/QSA interface on top of that ABI.
"""
from ._lib import LIB_PATH, QsaError, load  # noqa: F401

__all__ = ["LIB_PATH", "QsaError", "load"]
