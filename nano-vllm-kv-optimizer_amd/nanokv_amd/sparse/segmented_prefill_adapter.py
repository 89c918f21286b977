"""Segmented prefill adapter: scratch shared by the layers of one model, one stream.

Mirror of the reference's ``nanovllm/sparse/segmented_prefill_adapter.py``
(:50-159).  ``M12LayerRuntime.prefill_chunk`` hands the adapter the four
segments of a later chunk's keys -- the selected history blocks, the sink,
the previous recent window (logical order) and the chunk itself -- through
``prepare`` and gets the attention output from ``attend``
(m12_runtime.py:596-636).  The adapter owns no KV state and makes no
selection; its scratch is reused by every layer in turn, so the caller must
finish each layer on the adapter's stream before the next one prepares.

Backends:

* ``"flash_reuse"`` -- the segments are copied into one packed [S, Hkv, D]
  scratch (grown on demand, kept across layers and calls) and attended with
  bottom-right causal alignment (query t sees packed keys j <= S - T + t),
  the alignment of the reference's ``flash_attn_func(causal=True)``
  (segmented_prefill_adapter.py:139-144).  Here that attention is this
  library's packed kernel (``nkv_attend_packed``: the matrix-core kernel for
  long chunks, P rounded to bf16 for P.V as in flash attention).
* ``"operator"`` -- the reference loads a frozen external operator package
  (``llm_gpu_kernels``, segmented_prefill_adapter.py:16-38) that is not part
  of the reference repository; this package does not ship it, and constructing
  the adapter with it raises ``ValueError``.

Staging: the reference gathers the selected blocks into pinned host memory
and rejects pageable staging (:100-101).  Here the selected segment may be a
device tensor on the query's GPU (the default HBM history tier, whose blocks
never leave HBM) or pinned host memory (``history_tier="host"``); pageable
host memory is rejected with the reference's message.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..store import packed_attention


@dataclass(frozen=True)
class PrefillInvocation:
    """What ``prepare`` hands to ``attend`` (segmented_prefill_adapter.py:41-46):
    the queries, the four (k, v) segments as they sit in the scratch, the mode
    and the packed (k, v) views."""
    q: torch.Tensor
    segments: tuple
    mode: str
    packed: tuple | None


class SegmentedPrefillAdapter:
    """No KV state or selection ownership; the caller finishes each layer on one stream.

    Scratch is overwritten by the next ``prepare``; outputs are consumed
    before the next layer and not retained across invocations."""

    def __init__(self, backend, scale, geometry, operator_root=None):
        if backend not in ("flash_reuse", "operator"):
            raise ValueError("expected explicit experimental backend")
        if backend == "operator":
            raise ValueError("the 'operator' backend loads the external llm_gpu_kernels segmented operator, "
                             "which this package does not ship; use backend='flash_reuse' (the packed "
                             "matrix-core attention of this library)")
        self.backend, self.scale, self.geometry = backend, float(scale), geometry
        self.stream = torch.cuda.current_stream()
        self.device = self.stream.device
        self.packed_k = self.packed_v = self.selected_k = self.selected_v = None
        self.pack_capacity = self.selected_capacity = 0
        self.workspace = None
        self.workspace_builds = self.direct_calls = self.fa2_calls = 0
        self.selection_cache = {}
        self.module = self.policy = self.compile_cache = None
        self.provenance = None

    def _stream_check(self, device):
        if device != self.device or torch.cuda.current_stream(device).cuda_stream != self.stream.cuda_stream:
            raise ValueError("shared prefill scratch belongs to one CUDA device/stream")

    def precompile(self, tokens, lengths):
        """Mode that a chunk of `tokens` queries over segments of `lengths` takes
        (segmented_prefill_adapter.py:84-88); nothing is compiled at run time here."""
        return "fa2"

    def prepare(self, q, stage_k, stage_v, sink, recent, current):
        """Pack [selected | sink | recent | current] into the shared scratch
        (segmented_prefill_adapter.py:90-130)."""
        self._stream_check(q.device)
        lengths = (stage_k.shape[0], sink[0].shape[0], recent[0].shape[0], current[0].shape[0])
        if stage_k.shape != stage_v.shape or current[0].shape[0] != q.shape[0]:
            raise ValueError("inconsistent selected/current lengths")
        for t in (stage_k, stage_v):
            if t.device.type == "cpu":
                if not t.is_pinned():
                    raise ValueError("selected CPU staging must be pinned")
            elif t.device != q.device:
                raise ValueError("selected staging must be pinned host memory or on the query's device")
        _, heads, dim, dtype = self.geometry
        total = sum(lengths)
        if total > self.pack_capacity:
            self.pack_capacity = total
            self.packed_k = torch.empty((total, heads, dim), dtype=dtype, device=q.device)
            self.packed_v = torch.empty_like(self.packed_k)
            self.packed_k.record_stream(self.stream)
            self.packed_v.record_stream(self.stream)
        pk, pv = self.packed_k[:total], self.packed_v[:total]
        offset, segments = 0, []
        for length, (k, v) in zip(lengths, ((stage_k, stage_v), sink, recent, current)):
            dk, dv = pk[offset:offset + length], pv[offset:offset + length]
            dk.copy_(k, non_blocking=False)
            dv.copy_(v, non_blocking=False)
            segments.append((dk, dv))
            offset += length
        return PrefillInvocation(q, tuple(segments), "fa2", (pk, pv))

    def attend(self, invocation):
        """Bottom-right causal attention over the packed segments
        (segmented_prefill_adapter.py:132-147) -> [T, Hq, D]."""
        self._stream_check(invocation.q.device)
        self.fa2_calls += 1
        k, v = invocation.packed
        q = invocation.q
        return packed_attention(q, k, v, k.shape[0] - q.shape[0], self.scale)

    def stats(self):
        """Counters and scratch sizes (segmented_prefill_adapter.py:149-159)."""
        tensors = (self.packed_k, self.packed_v, self.selected_k, self.selected_v)
        scratch = sum(t.numel() * t.element_size() for t in tensors if t is not None)
        return dict(direct_calls=self.direct_calls, fa2_calls=self.fa2_calls,
                    workspace_builds=self.workspace_builds, shared_scratch_bytes=scratch,
                    direct_workspace_bytes=0, pack_capacity=self.pack_capacity,
                    selected_capacity=self.selected_capacity, cache=None)
