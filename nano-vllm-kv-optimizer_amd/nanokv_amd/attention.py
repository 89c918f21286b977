"""The caller side of the sparse layer-step.

``Attention`` routes a layer's post-RoPE q/k/v the way the reference's
``Attention.forward`` does in sparse mode (nanovllm/layers/attention.py:
64-99): verify mode -> ``verify_tokens``; the first prefill chunk -> dense
causal attention within the chunk, then ``prefill_first``; later prefill
chunks -> ``prefill_chunk``; one decode token -> ``decode``.  The reference
runs the first chunk through flash-attention; here it is
``M12LayerRuntime.dense_prefill`` on this library's matrix-core kernel.

``attach_m12_runtimes`` is the wiring of ``ModelRunner.allocate_kv_cache``
for the M12 runtime (nanovllm/engine/model_runner.py:125-183): every module
that has ``k_cache`` / ``v_cache`` gets a layer id, zero paged blocks and an
``M12LayerRuntime``.  All layers share one HBM store.

``Context`` / ``get_context`` / ``set_context`` / ``reset_context`` carry the
per-step batch description with the fields of nanovllm/utils/context.py, so a
model runner that sets the context before each forward drives both.

The dense paged-cache path of the reference (feature off) is not part of the
sparse layer-step; a layer without an enabled runtime raises.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from .sparse.m12_runtime import M12Config, M12LayerRuntime
from .store import SparseKVStore


@dataclass(slots=True)
class Context:
    """Per-step batch description (field names of nanovllm/utils/context.py:5-14)."""
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()


class Attention(nn.Module):
    """One attention layer's entry point (constructor of nanovllm/layers/attention.py:47-61)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.layer_id = None
        self.sparse_rt = None

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """q [T, Hq, D], k/v [T, Hkv, D] bf16 -> [T, Hq, D] bf16."""
        context = get_context()
        rt = self.sparse_rt
        if rt is None or not rt.enabled:
            raise NotImplementedError(
                "dense paged attention (sparse runtime off) is not part of nanokv_amd: "
                "attach an M12LayerRuntime as sparse_rt (attach_m12_runtimes)")
        if rt.verify_mode:
            return rt.verify_tokens(q, k, v, q.device)
        assert q.shape[0] == (context.max_seqlen_q or q.shape[0]) or context.is_prefill
        if context.is_prefill:
            if rt.prefill_len == 0:
                o = rt.dense_prefill(q, k, v, scale=self.scale)
                rt.prefill_first(q, k, v)
                return o
            return rt.prefill_chunk(q, k, v, q.device)
        assert q.shape[0] == 1, "sparse decode supports a single query token"
        assert context.block_tables is None, "sparse decode must not use paged block tables"
        assert self.k_cache.numel() == 0, "sparse mode must allocate zero paged blocks"
        return rt.decode(q, k, v, q.device)


def attach_m12_runtimes(model: nn.Module, cfg: M12Config, device=None) -> list[M12LayerRuntime]:
    """Give every attention module of `model` its layer id, zero paged blocks and an
    M12LayerRuntime over one shared HBM store (model_runner.py:125-183)."""
    layers = [m for m in model.modules() if hasattr(m, "k_cache") and hasattr(m, "v_cache")]
    if not layers:
        raise ValueError("model has no attention modules (nothing with k_cache / v_cache)")
    B = cfg.block_size
    store = SparseKVStore(
        len(layers), num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
        block_size=B, r=cfg.r, cap_blocks=(cfg.max_model_len + B - 1) // B,
        sink_tokens=cfg.sink_tokens, recent_tokens=cfg.recent_tokens, kv_format=cfg.kv_format,
        device=device, history_tier=cfg.history_tier)
    runtimes = []
    for layer_id, module in enumerate(layers):
        module.layer_id = layer_id
        module.k_cache = torch.empty(0)
        module.v_cache = torch.empty(0)
        module.sparse_rt = M12LayerRuntime(layer_id, cfg, store=store)
        runtimes.append(module.sparse_rt)
    return runtimes


__all__ = ["Attention", "Context", "attach_m12_runtimes", "get_context", "reset_context", "set_context"]
