"""Sparse-attention runtime (mirror of the reference's ``nanovllm.sparse`` M12 surface)."""

from .m12_runtime import (  # noqa: F401
    M12Config,
    M12LayerRuntime,
    M12ModelRuntime,
    dynamic_top_k_from_scores,
    prefill_query_summaries,
    prefill_recent_slice,
)
