"""nanokv_amd: MI355X-native NanoKV sparse-attention layer-step.

The hot path (block scoring, Top-K selection, in-place gather of selected /
sink / recent K/V and segmented GQA attention, with optional int8 history)
runs as hand-written gfx950 HIP kernels in ``libnanokv.so`` behind the C ABI
of ``include/nanokv.h``.  ``nanokv_amd.sparse.m12_runtime`` mirrors the
reference's ``nanovllm.sparse.m12_runtime`` call surface.
"""

from . import _lib  # noqa: F401

__all__ = ["_lib"]
