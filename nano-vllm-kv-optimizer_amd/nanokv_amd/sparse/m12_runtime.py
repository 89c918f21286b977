"""MI355X-native M12 sparse layer runtime.

Drop-in for ``nanovllm/sparse/m12_runtime.py`` of the reference: the same
``M12Config`` fields and validation errors, and an ``M12LayerRuntime`` with
the same call surface (``decode``, ``prefill_first``, ``prefill_chunk``,
``verify_tokens``, ``commit_verified``, ``rollback_verified``, ``reset``,
``reserve_blocks``, ``_gpu_select``, ``_gpu_select_per_query``,
``_fused_attention``, ``_prefill_attention``, ``_build_reps_gpu``) and state
attributes (``nblocks_filled``,
``valid_len``, ``prefill_len``, ``reps_gpu``, ``protected_blocks``,
``last_block_ids``, ``timings`` ...), so ``Attention.forward``
(nanovllm/layers/attention.py:64-99) and the engine wiring
(nanovllm/engine/model_runner.py:134-184) can use it unchanged.

What differs by design: the history stays in HBM (no host gather, no H2D
pack); selected block ids stay on the device during decode and are copied to
the host only when ``last_block_ids`` / ``ids_history`` is read; every
operation is a hand-written gfx950 HIP kernel behind the C ABI of
include/nanokv.h.  ``M12ModelRuntime`` runs the same kernels for all layers of
a model in one launch per stage.
"""

from __future__ import annotations

import ctypes
import math
from contextlib import nullcontext
from dataclasses import dataclass
from time import perf_counter

import torch

from .. import _lib
from ..store import SparseKVStore, current_stream_ptr, packed_attention, query_summaries, tile_summaries

# Query rows per group of the few-query kernels: one 16-column MFMA tile, or
# two (the wide kernel) once a chunk's rows exceed one tile.
TILE_ROWS = 16
WIDE_ROWS = 32


def few_query_group(tq: int, g: int) -> int:
    """Queries per group of the few-query attention (the C side's group_shape)."""
    rows = WIDE_ROWS if tq * g > TILE_ROWS else TILE_ROWS
    return min(tq, max(1, rows // g))


# ---------------------------------------------------------------------------
# Host-side helpers (same contracts as the reference's module functions)
# ---------------------------------------------------------------------------


def prefill_recent_slice(valid_len: int, sink_tokens: int, recent_tokens: int):
    """(buffer_start, buffer_offset, length) of the recent buffer not also sink.

    Reference: m12_runtime.py:32-50.
    """
    assert valid_len >= 0
    assert sink_tokens >= 0
    assert recent_tokens >= 0
    sink_len = min(sink_tokens, valid_len)
    buffer_len = min(recent_tokens, valid_len)
    buffer_start = valid_len - buffer_len
    include_start = max(sink_len, buffer_start)
    return buffer_start, include_start - buffer_start, valid_len - include_start


def prefill_query_summaries(q: torch.Tensor, nsegments: int) -> torch.Tensor:
    """Segment means of a prefill chunk's queries, [nseg, Hq, D] bf16, on device.

    Reference: m12_runtime.py:53-67 (``q.mean(dim=0, keepdim=True)`` for one
    segment, ``tensor_split`` means otherwise).  Each mean is the bf16
    round-to-nearest-even of the exact mean.
    """
    assert q.ndim == 3, "q must be [T, Hq, D]"
    assert nsegments > 0
    return query_summaries(q.unsqueeze(0).contiguous(), nsegments)[0]


def dynamic_top_k_from_scores(top_scores: torch.Tensor, max_k: int, target_mass: float) -> int:
    """Decode budget from half, three quarters or all candidates.

    Reference: m12_runtime.py:70-95 (host-side, CPU scores).
    """
    assert top_scores.ndim == 1 and top_scores.device.type == "cpu"
    assert 0.0 < target_mass <= 1.0 and max_k > 0
    count = top_scores.numel()
    if count < max_k or count <= 1 or not bool(torch.isfinite(top_scores).all()):
        return count
    scale = top_scores.std(unbiased=False)
    if float(scale) <= 1e-6:
        return count
    weights = torch.softmax((top_scores - top_scores[0]) / scale, dim=0)
    cumulative = weights.cumsum(dim=0)
    choices = sorted({max(1, (max_k + 1) // 2), max(1, (3 * max_k + 3) // 4), max_k})
    for choice in choices:
        if float(cumulative[choice - 1]) >= target_mass:
            return choice
    return max_k


@dataclass
class M12Config:
    """Same fields, defaults and validation as the reference (m12_runtime.py:98-166).

    Extra fields (no reference counterpart): ``quant_scale_layout`` ("channel_block" = the
    reference's K-per-channel / V-per-block fp32 scales, "token" = per-token
    per-KV-head fp16 scales) and ``attend_splits`` (workgroups per KV head in
    the attention kernel; None = automatic) and ``mfma_chunk_min_tokens``
    (prefill / verify chunks of at least this many queries use the
    matrix-core kernel, shorter ones the few-query kernel; None = automatic:
    the matrix-core kernel as soon as the chunk's query rows, tokens x heads
    per KV head, exceed the few-query kernels' widest group of 32 rows, which
    they would otherwise split, reading every block once per group),
    ``history_tier``
("hbm": the whole history in HBM; "host": hist_k / hist_v in pinned host
memory, read in place by the same kernels over the host link, the
reference's offload mode without its gather and H2D copy).  ``use_index_select``,
    ``decode_kv_pipeline`` and ``gather_sort``'s gather-locality purpose
    belong to the host-offload design and do not change the HBM path
    (``gather_sort`` still orders ``last_block_ids`` ascending).
    ``prefill_selection`` ("chunk": one selection per prefill chunk, the
    reference's routing; "tile": one per tile of ``prefill_selection_tile``
    queries, from each tile's bf16 query mean -- no reference counterpart;
    the tile must be a multiple of 128 / (num_heads / num_kv_heads) tokens).
    """
    block_size: int = 64
    r: int = 4
    recent_tokens: int = 512
    sink_tokens: int = 64
    top_k_blocks: int = 32
    prefill_top_k_blocks: int | None = None
    decode_top_k_blocks: int | None = None
    dynamic_top_k: bool = False
    dynamic_top_k_mass: float = 0.90
    decode_relative_a: float | None = None
    decode_relative_max_blocks: int = 48
    decode_relative_union: bool = False
    decode_query_window: int = 1
    fused_selector: bool = False
    quant_history: bool = False
    verify_union_blocks: int = 0
    fused_dequant: bool = False
    gather_sort: bool = False
    max_model_len: int = 131072
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    dtype: torch.dtype = torch.bfloat16
    scale: float = 128.0 ** -0.5
    use_index_select: bool = True
    decode_kv_pipeline: bool = False
    selector_cuda_graph: bool = False
    selector_static_mask: bool = False
    check_finite_outputs: bool = False
    prefill_query_segments: int = 1
    prefill_attention_backend: str = "torch"
    prefill_adapter: object | None = None
    quant_scale_layout: str = "channel_block"
    attend_splits: int | None = None
    mfma_chunk_min_tokens: int | None = None
    history_tier: str = "hbm"
    prefill_selection: str = "chunk"
    prefill_selection_tile: int = 64

    def __post_init__(self):
        if self.decode_kv_pipeline and not self.use_index_select:
            raise ValueError("decode_kv_pipeline requires use_index_select")
        for name, budget in (
            ("prefill_top_k_blocks", self.prefill_top_k_blocks),
            ("decode_top_k_blocks", self.decode_top_k_blocks),
        ):
            if budget is not None and not 1 <= budget <= self.top_k_blocks:
                raise ValueError(f"{name} must be in [1, top_k_blocks]")
        if self.decode_relative_a is not None:
            if not 0.0 < self.decode_relative_a < 1.0:
                raise ValueError("decode_relative_a must be in (0, 1)")
            if self.decode_relative_max_blocks < 1:
                raise ValueError("decode_relative_max_blocks must be >= 1")
        if self.decode_query_window < 1:
            raise ValueError("decode_query_window must be >= 1")
        if self.fused_dequant and not self.quant_history:
            raise ValueError("fused_dequant requires quant_history")
        if self.quant_scale_layout not in ("channel_block", "token"):
            raise ValueError("quant_scale_layout must be 'channel_block' or 'token'")
        if self.attend_splits is not None and not 1 <= self.attend_splits <= 64:
            raise ValueError("attend_splits must be in [1, 64]")
        if self.mfma_chunk_min_tokens is not None and self.mfma_chunk_min_tokens < 1:
            raise ValueError("mfma_chunk_min_tokens must be >= 1 or None")
        if self.history_tier not in ("hbm", "host"):
            raise ValueError("history_tier must be 'hbm' or 'host'")
        if self.prefill_selection not in ("chunk", "tile"):
            raise ValueError("prefill_selection must be 'chunk' or 'tile'")
        if self.prefill_selection_tile < 1:
            raise ValueError("prefill_selection_tile must be >= 1")

    @property
    def kv_format(self) -> str:
        if not self.quant_history:
            return "bf16"
        return "int8" if self.quant_scale_layout == "channel_block" else "int8_token"


def _check_hip_shapes(cfg: M12Config) -> None:
    if cfg.dtype != torch.bfloat16:
        raise ValueError("the HIP runtime computes on bfloat16 K/V/q (cfg.dtype must be torch.bfloat16)")
    if cfg.head_dim != 128 or cfg.block_size != 64:
        raise ValueError("the gfx950 kernels are built for head_dim=128 and block_size=64")
    if cfg.num_heads % cfg.num_kv_heads or cfg.num_heads // cfg.num_kv_heads not in (1, 2, 4, 8, 16):
        raise ValueError("num_heads / num_kv_heads must be 1, 2, 4, 8 or 16")
    if cfg.r not in (1, 2, 4, 8):
        raise ValueError("r must be 1, 2, 4 or 8")
    tpw = 128 // (cfg.num_heads // cfg.num_kv_heads)
    if cfg.prefill_selection == "tile" and cfg.prefill_selection_tile % tpw:
        raise ValueError(f"prefill_selection_tile must be a multiple of {tpw} tokens for this head shape")


# ---------------------------------------------------------------------------
# Sequence bookkeeping + kernel calls over a range of layers
# ---------------------------------------------------------------------------


class _SparseCore:
    """One sequence's sparse-attention state over layers [layer0, layer0 + nl).

    Bookkeeping follows M12LayerRuntime (m12_runtime.py:169-1346); the data
    lives in a SparseKVStore.  All layers of the range share lengths,
    protected set and ring position, which is what a model's layers see.
    """

    def __init__(self, cfg: M12Config, store: SparseKVStore, layer0: int, nl: int):
        self.cfg = cfg
        self.store = store
        self.layer0 = layer0
        self.nl = nl
        self.device = store.device
        self.max_blocks = store.cap_blocks
        self.valid_len = 0
        self.prefill_len = 0
        self.nblocks_filled = 0
        self.ring_start = 0
        self.protected_blocks: set[int] = set()
        self.k_scale_set = False
        self.pending = None
        self._prot_key = None
        self._prot_dev = None
        self._ws: dict[str, torch.Tensor] = {}
        self._ring_dev = None       # int32 [nl]: ring starts in device memory (device-ring decode)
        self._ring_dev_pos = None   # the value every entry of _ring_dev holds

    # -- workspaces ---------------------------------------------------------
    def _buf(self, name: str, numel: int, dtype) -> torch.Tensor:
        t = self._ws.get(name)
        if t is None or t.numel() < numel or t.dtype != dtype:
            t = torch.empty(max(numel, 1), dtype=dtype, device=self.device)
            self._ws[name] = t
        return t[:numel]

    def _zeroed_keys(self, numel: int, ws: str = "") -> torch.Tensor:
        """Score-key workspace: zero before first use, left zero by every select."""
        t = self._ws.get("keys" + ws)
        if t is None or t.numel() < numel:
            t = torch.zeros(max(numel, 1), dtype=torch.int32, device=self.device)
            self._ws["keys" + ws] = t
        return t[:numel]

    def reset(self) -> None:
        self.valid_len = 0
        self.prefill_len = 0
        self.nblocks_filled = 0
        self.protected_blocks.clear()
        self.k_scale_set = False
        self.pending = None
        self._prot_key = None

    # -- store (m12_runtime.py:420-513) --------------------------------------
    def store_kv(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: [nl, T, Hkv, D] bf16 device tensors."""
        cfg = self.cfg
        B, R = cfg.block_size, cfg.recent_tokens
        T = k.shape[1]
        assert T >= 2
        k = k.contiguous()
        v = v.contiguous()
        nblk = (T + B - 1) // B
        start = self.nblocks_filled
        need = start + nblk
        if need > self.max_blocks:
            raise ValueError(f"history of {need} blocks exceeds max_model_len "
                             f"({self.max_blocks} blocks)")
        compute_k_scale = cfg.kv_format == "int8" and not self.k_scale_set
        self.store.store_chunk(self.layer0, k, v, start, compute_k_scale, self.prefill_len == 0)
        self.k_scale_set = self.k_scale_set or compute_k_scale
        self.store.build_reps(self.layer0, k, start)
        recent_len = min(R, self.valid_len + T)
        if T >= recent_len:
            self.store.recent_update(self.layer0, self.nl, k, v, T - recent_len, recent_len,
                                     self.ring_start, 0, 0)
        else:
            carry = recent_len - T
            old = min(R, self.valid_len)
            self.store.recent_update(self.layer0, self.nl, k, v, 0, T, self.ring_start, old, carry)
        self.valid_len += T
        self.prefill_len += T
        self.nblocks_filled = need
        n_recent_blocks = R // B
        self.protected_blocks = {0} | set(range(max(1, need - n_recent_blocks), need))

    def commit(self, n: int) -> None:
        """commit_verified (m12_runtime.py:777-803)."""
        if n <= 0:
            self.pending = None
            return
        k, v = self.pending
        T = int(n)
        R = self.cfg.recent_tokens
        old = min(R, self.valid_len)
        new = min(R, self.valid_len + T)
        if T >= R:
            self.store.recent_update(self.layer0, self.nl, k, v, T - R, R, self.ring_start, 0, 0)
        else:
            carry = new - T
            self.store.recent_update(self.layer0, self.nl, k, v, 0, T, self.ring_start, old, carry)
        self.valid_len += T
        self.pending = None

    # -- selection (m12_runtime.py:959-1087) ---------------------------------
    def protected_dev(self):
        nb = self.nblocks_filled
        ids = tuple(sorted(p for p in self.protected_blocks if 0 <= p < nb))
        if ids != self._prot_key:
            self._prot_dev = torch.tensor(list(ids) or [0], dtype=torch.int32, device=self.device)
            self._prot_key = ids
        return self._prot_dev, len(ids)

    def effective_k(self, requested: int) -> int:
        nb = self.nblocks_filled
        n_prot = len([p for p in self.protected_blocks if 0 <= p < nb])
        return min(int(requested), max(1, nb - n_prot))

    def select(self, q: torch.Tensor, requested: int, *, per_query: bool = False,
               order: int = _lib.NKV_ORDER_SCORE_DESC, lo: int = 0, ws: str = "",
               ids_out: torch.Tensor | None = None):
        """q: [nl, nq, Hq, D] bf16 -> (ids [nl, nq', requested] int32, vals, k_eff).

        lo: first layer of q relative to this core's range; ws tags the
        workspaces (calls in flight together on different streams need their
        own); ids_out: optional destination for the ids."""
        nb = self.nblocks_filled
        if nb <= 0:
            raise ValueError("selection needs at least one history block")
        if requested < 1:
            raise ValueError("the block budget must be >= 1")
        q = q.contiguous()
        nl, nq = q.shape[0], q.shape[1]
        nqo = nq if per_query else 1
        prot, n_prot = self.protected_dev()
        keys = self._zeroed_keys(nl * nqo * nb, ws)
        scores = self._buf("scores" + ws, nl * nqo * nb, torch.float32)
        if ids_out is None:
            ids = self._buf("ids" + ws, nl * nqo * requested, torch.int32).view(nl, nqo, requested)
        else:
            ids = ids_out
        vals = self._buf("vals" + ws, nl * nqo * requested, torch.float32).view(nl, nqo, requested)
        self.store.select(self.layer0 + lo, q, nb, prot, n_prot, requested, order, per_query,
                          keys, scores, ids, vals)
        self._last_scores = scores.view(nl, nqo, nb)
        return ids, vals, self.effective_k(requested)

    # per-query Top-K and union in one launch (36-layer 16K verify round: one
    # launch fewer between the scorer and the attention)
    FUSED_SELECT_UNION = True

    def select_per_query_union(self, q: torch.Tensor, requested: int):
        """Per-query selection and its union for every layer (m12_runtime.py:1057-1087):
        q [nl, nq, Hq, D] -> (union [nl, umax] ascending then -1, counts [nl],
        allowed [nl, nq, umax] uint8).  One launch for the Top-K and the union
        (nkv_select_per_query, umax = nq * min(requested, nblocks)) where its
        limits allow, else nkv_select + nkv_select_union (umax = nq * k_eff)."""
        nb = self.nblocks_filled
        if nb <= 0:
            raise ValueError("selection needs at least one history block")
        if requested < 1:
            raise ValueError("the block budget must be >= 1")
        q = q.contiguous()
        nl, nq = q.shape[0], q.shape[1]
        fused = self.FUSED_SELECT_UNION and nq <= 16 and requested <= 64 and nb <= 2048
        kk = self.effective_k(requested)
        umax = nq * (min(requested, nb) if fused else kk)
        union = self._buf("union", nl * umax, torch.int32).view(nl, umax)
        count = self._buf("union_count", nl, torch.int32)
        allowed = self._buf("allowed", nl * nq * umax, torch.uint8).view(nl, nq, umax)
        if fused:
            prot, n_prot = self.protected_dev()
            keys = self._zeroed_keys(nl * nq * nb, "")
            scores = self._buf("scores", nl * nq * nb, torch.float32)
            ids = self._buf("ids", nl * nq * requested, torch.int32).view(nl, nq, requested)
            vals = self._buf("vals", nl * nq * requested, torch.float32).view(nl, nq, requested)
            self.store.select_per_query(self.layer0, q, nb, prot, n_prot, requested, keys, scores, ids, vals,
                                        umax, union, count, allowed)
            self._last_scores = scores.view(nl, nq, nb)
        else:
            ids, _, kk = self.select(q, requested, per_query=True)
            self.store.select_union(ids, kk, umax, union, count, allowed)
        return union, count, allowed, umax

    # -- attention ------------------------------------------------------------
    # the stream form pays off once every resident wavefront gets a couple of
    # segments (one round of ~2048 wavefronts on an MI355X)
    STREAM_MIN_SEGMENTS = 4096
    # the wide kernel's tiered plan pays off once the groups alone fill a
    # quarter of the device's workgroup slots (36 layers x 8 KV heads = 288)
    WIDE_PLAN_MIN_GROUPS = 128

    def _splits(self, nseg: int, nqg: int, rows: int = 4) -> int:
        """Attention split count for nseg segments per (layer, KV head, query
        group); rows = query rows per group (17-32: the wide few-query kernel).
        0 = the 4-row kernel's stream form: one resident round of wavefronts
        shares the launch's whole segment list evenly (no second, partly
        filled round of workgroups, no wavefront idling at its workgroup's
        merge); for the wide kernel, its tiered plan: two rounds of
        workgroups, large pieces of the first groups' segments, then small
        pieces of the rest's (no partly filled last round)."""
        if self.cfg.attend_splits is not None:
            return self.cfg.attend_splits
        if rows <= 4 and self.nl * self.store.num_kv_heads * nqg * nseg >= self.STREAM_MIN_SEGMENTS:
            return 0
        if 16 < rows <= 32 and self.nl * self.store.num_kv_heads * nqg >= self.WIDE_PLAN_MIN_GROUPS:
            return 0
        # Workgroups per launch measured best on the 36-layer 32K decode step
        # (tok/s, splits 2 / 3 / 5 / 6 / 7 / 9): bf16 ~1440 (8382 / 8827 /
        # 9261 / 9141 / 8992 / 8838); both int8 forms, whose segments carry
        # half the bytes, ~900 (per-block 9434 / 10122 / 9792 / 9555 / 9347 /
        # 8959, per-token 9378 / 9929 / 9831 / 9766 / 9615 / 9385).  Never
        # more than one segment per wavefront.
        # Workgroups go round-robin over the 8 XCDs with the split index
        # fastest, so a split count with a factor 4 in common with 8 pins
        # the splits that carry an extra segment to the same XCDs (4 and 8
        # splits measured 5% and 14% slower than 5 in bf16): such counts
        # move up by one.
        # The wide few-query kernel (verify's draft tokens, 17-32 rows a
        # group) holds two workgroups per CU: ~900 as well (36-layer 16K
        # verify, 6 tokens, bf16, us per round at splits 1 / 2 / 3 / 4 / 5 / 6
        # / 7 / 9: 372 / 398 / 344.7 / 370 / 353 / 367 / 363 / 380).
        target = 1440 if self.cfg.kv_format == "bf16" and rows <= 16 else 900
        want = max(1, round(target / (self.store.num_kv_heads * self.nl * nqg)))
        cap = max(1, min(-(-nseg // 4), 64))
        s = min(want, cap)
        if s > 1 and s % 4 == 0:
            s = s + 1 if s < cap else s - 1
        return s

    def _prefill_splits(self, tq: int, nseg: int) -> int:
        """Split-K for the matrix-core kernel: about 1536 workgroups per launch
        when the query tiles alone give far fewer (short chunks, verify), each
        split keeping at least 4 segments.  Measured on the 36-layer 16K
        verify round (6 queries): 417 us at ~1536 workgroups (5 splits) vs
        427 at ~1024, 419 at ~2048, 432 at ~3072."""
        g = self.cfg.num_heads // self.cfg.num_kv_heads
        tiles = -(-tq // (128 // g)) * self.store.num_kv_heads * self.nl
        want = max(1, round(1536 / tiles))
        return max(1, min(want, nseg // 4, 64))

    def attend(self, q, k_new, v_new, *, n_chunk, write_slot, ids, ids_stride,
               n_hist, allowed, sink_len, ring_base, rec_lo, rec_len, lo=0, ws="", out=None,
               allowed_stride=0, scale=None):
        cfg = self.cfg
        scale = cfg.scale if scale is None else scale
        nl, tq = q.shape[0], q.shape[1]
        g = cfg.num_heads // cfg.num_kv_heads
        qpg = few_query_group(tq, g)
        nqg = -(-tq // qpg)
        R = cfg.recent_tokens
        nseg = n_hist + -(-sink_len // 64) + (-(-R // 64) if rec_len else 0) + -(-n_chunk // 64)
        splits = self._splits(nseg, nqg, min(qpg, tq) * g)
        if out is None:
            out = torch.empty_like(q)
        part = self._buf("partial" + ws, self.store.attend_workspace_floats(nl, tq, splits), torch.float32)
        self.store.attend(self.layer0 + lo, q, k_new, v_new, n_chunk, write_slot, ids,
                          ids_stride, n_hist, allowed, sink_len, ring_base, rec_lo, rec_len,
                          scale, splits, part, out, allowed_stride)
        return out

    def decode_attend(self, q, k, v, ids, ids_stride, n_hist, *, lo=0, ws="", out=None,
                      advance=True):
        """Decode step 1 + 3-5 (m12_runtime.py:1164-1320): q [nl,1,Hq,D], k/v [nl,1,Hkv,D].

        lo / ws / out: layer sub-range, workspace tag and output destination
        (see select); advance=False leaves the ring position and length for
        advance_decode()."""
        w = self.decode_window()
        out = self.attend(q.contiguous(), k.contiguous(), v.contiguous(), n_chunk=1,
                          write_slot=w["write_slot"], ids=ids,
                          ids_stride=ids_stride, n_hist=n_hist, allowed=None,
                          sink_len=w["sink_len"], ring_base=w["ring_base"],
                          rec_lo=w["rec_lo"], rec_len=w["rec_len"], lo=lo, ws=ws, out=out)
        if advance:
            self.advance_decode()
        return out, w["sink_len"], w["rec_len"] + 1

    def decode_window(self) -> dict:
        """Segments of this step's decode attention.  The logical recent window
        after the shift is [R - rec_len, R); its last slot is the new token,
        attended as a one-token chunk and stored into the freed physical slot
        (the old logical slot 0), so the ring part is the rec_len - 1 before it."""
        cfg = self.cfg
        R = cfg.recent_tokens
        rec_len = min(R, self.valid_len + 1)
        return {"sink_len": min(cfg.sink_tokens, self.valid_len), "write_slot": self.ring_start,
                "ring_base": (self.ring_start + 1) % R, "rec_lo": R - rec_len,
                "rec_len": rec_len - 1}

    def decode_splits(self, n_hist: int) -> int:
        """The attention split count decode_attend uses for n_hist selected blocks."""
        w = self.decode_window()
        B, R = self.cfg.block_size, self.cfg.recent_tokens
        nseg = n_hist + -(-w["sink_len"] // B) + (-(-R // B) if w["rec_len"] else 0) + 1
        return self._splits(nseg, 1)

    def advance_decode(self) -> None:
        """The decode token is in the ring: move the ring start, grow the length."""
        self.ring_start = (self.ring_start + 1) % self.cfg.recent_tokens
        self.valid_len += 1

    # -- device-ring decode (capturable in a HIP graph) ----------------------------
    def decode_ring_ready(self) -> bool:
        """Steady decode: sink and recent window full, so every argument of a
        decode step except the ring position repeats from step to step."""
        return (self.nblocks_filled > 0 and self.valid_len + 1 >= self.cfg.recent_tokens
                and self.valid_len >= self.cfg.sink_tokens)

    def decode_ring(self, q, k, v, requested: int, *, out=None):
        """The decode step through nkv_decode_step_ring: q [nl,1,Hq,D], k/v [nl,1,Hkv,D].

        The ring start lives in a device array that the call advances, so the
        enqueued work is the same every step and can be captured and
        replayed; advance_ring() is the host side of each replay.  Returns
        (out, ids [nl,1,requested], n_hist, window)."""
        if not self.decode_ring_ready():
            raise RuntimeError("device-ring decode needs a full sink and recent window")
        if self._ring_dev is None:
            self._ring_dev = torch.empty(self.nl, dtype=torch.int32, device=self.device)
            self._ring_dev_pos = None
        if self._ring_dev_pos != self.ring_start:   # the host moved the ring since (or never synced)
            self._ring_dev.fill_(self.ring_start)
            self._ring_dev_pos = self.ring_start
        nb = self.nblocks_filled
        n_hist = self.effective_k(requested)
        w = self.decode_window()
        splits = self.decode_splits(n_hist)
        prot, n_prot = self.protected_dev()
        keys = self._zeroed_keys(self.nl * nb, "/ring")
        ids = self._buf("ids/ring", self.nl * requested, torch.int32).view(self.nl, 1, requested)
        part = self._buf("partial/ring", self.store.attend_workspace_floats(self.nl, 1, splits), torch.float32)
        if out is None:
            out = torch.empty_like(q)
        self.store.decode_step_ring(self.layer0, q.contiguous(), k.contiguous(), v.contiguous(), nb, prot, n_prot,
                                    requested, n_hist, w["sink_len"], self._ring_dev, self.cfg.scale, splits, keys,
                                    ids, part, out)
        self.advance_ring()
        return out, ids, n_hist, w

    def advance_ring(self) -> None:
        """Host bookkeeping of one device-ring decode step (the device array moved itself)."""
        self.advance_decode()
        self._ring_dev_pos = self.ring_start

    def select_tiles(self, q, requested: int, tile: int, order: int = _lib.NKV_ORDER_SCORE_DESC):
        """Per-query-tile selection of a prefill chunk: q [nl, T, Hq, D] ->
        (ids [nl, ntiles, requested] int32, k_eff).  Tile i's routing query is
        the bf16 mean of queries [i * tile, min(T, (i + 1) * tile)) (the
        reference's query summary, m12_runtime.py:53-67, per tile), selected
        with the chunk's protected set and budget."""
        nl, T = q.shape[0], q.shape[1]
        ntiles = -(-T // tile)
        if ntiles > 64:
            raise ValueError(f"per-tile prefill selection supports at most 64 tiles per chunk "
                             f"(got {ntiles} tiles of {tile} tokens)")
        summ = tile_summaries(q, tile)
        ids, _, k_eff = self.select(summ, requested, per_query=True, order=order, ws="/tiles")
        return ids, k_eff

    def chunk_attend_tiled(self, q, k, v, ids, tile: int, n_hist: int, scale=None):
        """chunk_attend with one history selection per tile of `tile` queries:
        ids [nl, ntiles, K] (nkv_prefill_attend_tiled; chunks too short for the
        matrix-core kernel are one tile and take chunk_attend)."""
        cfg = self.cfg
        scale = cfg.scale if scale is None else float(scale)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        tq, g = q.shape[1], cfg.num_heads // cfg.num_kv_heads
        ids = ids.contiguous()
        if tq <= tile and not self._uses_mfma(tq):
            return self.chunk_attend(q, k, v, ids, ids.shape[1] * ids.shape[2], n_hist, scale=scale)
        sink_len = min(cfg.sink_tokens, self.valid_len)
        _, off, ln = prefill_recent_slice(self.valid_len, cfg.sink_tokens, cfg.recent_tokens)
        out = torch.empty_like(q)
        B = cfg.block_size
        nseg = n_hist + -(-sink_len // B) + (-(-cfg.recent_tokens // B) if ln else 0) + -(-tq // B)
        splits = self._prefill_splits(tq, nseg)
        part = None
        if splits > 1:
            part = self._buf("pf_partial", self.store.prefill_workspace_floats(self.nl, tq, splits), torch.float32)
        self.store.prefill_attend_tiled(self.layer0, q, k, v, ids, ids.shape[1] * ids.shape[2], ids.shape[2],
                                        tile, n_hist, sink_len, self.ring_start, off, ln, scale, out, splits, part)
        return out, sink_len, ln

    def _uses_mfma(self, tq: int) -> bool:
        """Whether a chunk of tq queries takes the matrix-core kernel: its query
        rows (tq x heads per KV head) exceed the widest few-query group, or
        cfg.mfma_chunk_min_tokens says so."""
        cfg = self.cfg
        if cfg.mfma_chunk_min_tokens is not None:
            return tq >= cfg.mfma_chunk_min_tokens
        return tq * (cfg.num_heads // cfg.num_kv_heads) > WIDE_ROWS

    def chunk_attend(self, q, k, v, ids, ids_stride, n_hist, allowed=None, allowed_stride=0,
                     scale=None):
        """[selected | sink | previous recent | chunk (causal)] (m12_runtime.py:592-639, :725-758).

        allowed: uint8 [tq, n_hist] shared by the layers, or per layer with
        layer stride allowed_stride.  scale: softmax scale (default cfg.scale).
        With nothing stored yet (valid_len 0, n_hist 0) this is plain causal
        attention within the chunk."""
        cfg = self.cfg
        scale = cfg.scale if scale is None else float(scale)
        sink_len = min(cfg.sink_tokens, self.valid_len)
        _, off, ln = prefill_recent_slice(self.valid_len, cfg.sink_tokens, cfg.recent_tokens)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        tq = q.shape[1]
        if self._uses_mfma(tq):
            out = torch.empty_like(q)
            B = cfg.block_size
            nseg = n_hist + -(-sink_len // B) + (-(-cfg.recent_tokens // B) if ln else 0) + -(-tq // B)
            splits = self._prefill_splits(tq, nseg)
            part = None
            if splits > 1:
                part = self._buf("pf_partial", self.store.prefill_workspace_floats(self.nl, tq, splits),
                                 torch.float32)
            self.store.prefill_attend(self.layer0, q, k, v, ids, ids_stride, n_hist, allowed,
                                      sink_len, self.ring_start, off, ln, scale, out,
                                      allowed_stride, splits, part)
        else:
            out = self.attend(q, k, v, n_chunk=q.shape[1], write_slot=-1, ids=ids,
                              ids_stride=ids_stride, n_hist=n_hist, allowed=allowed,
                              sink_len=sink_len, ring_base=self.ring_start, rec_lo=off,
                              rec_len=ln, allowed_stride=allowed_stride, scale=scale)
        return out, sink_len, ln


# ---------------------------------------------------------------------------
# Per-layer runtime (the reference's class surface)
# ---------------------------------------------------------------------------


class M12LayerRuntime:
    """Per-layer sparse runtime on the HBM store (m12_runtime.py:169-1346)."""

    def __init__(self, layer_id: int, cfg: M12Config, *, store: SparseKVStore | None = None,
                 store_layer: int | None = None, device=None):
        _check_hip_shapes(cfg)
        self.layer_id = layer_id
        self.cfg = cfg
        self.enabled = True
        B = cfg.block_size
        self.max_blocks = (cfg.max_model_len + B - 1) // B
        self.groups_per_kv = cfg.num_heads // cfg.num_kv_heads
        if store is None:
            store = SparseKVStore(
                1, num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                block_size=B, r=cfg.r, cap_blocks=self.max_blocks, sink_tokens=cfg.sink_tokens,
                recent_tokens=cfg.recent_tokens, kv_format=cfg.kv_format, device=device,
                history_tier=cfg.history_tier)
            store_layer = 0
        elif store_layer is None:
            store_layer = layer_id
        self.store = store
        self.store_layer = store_layer
        self._core = _SparseCore(cfg, store, store_layer, 1)
        self.quant_history = cfg.quant_history
        # [Hkv, max_blocks, r, D] view of this layer's representatives
        self.reps_gpu = store.reps[store_layer]
        self.timings: dict[str, float] = {}
        self.last_prefill_query_summaries = 0
        self.prefill_cpu_gather_ms = 0.0
        self.record_ids = False
        self.ids_history: list[list[int]] = []
        self.record_q = False
        self.q_history: list[torch.Tensor] = []
        self.verify_mode = False
        self.verify_lossless = False
        # decode through nkv_decode_step_ring once the window is full (same
        # results; the ring position lives on the device, so a decode step can
        # be captured in a HIP graph and replayed); host-side selection rules,
        # gather_sort and query windows keep the regular path
        self.device_ring = False
        self.last_verify_timings: dict = {}
        # selector graph (use_graph): one captured score + top-k per sequence
        # and shape; _reps_version moves whenever representatives are rebuilt
        self._selector_graph = None
        self._selector_graph_key = None
        self._selector_graph_q = None
        self._selector_graph_outputs = None
        self._selector_graph_keep = None
        self._reps_version = 0
        self.selector_graph_setup_ms = 0.0
        self.selector_graph_builds = 0
        self.profile_cuda_stages = False
        self.profile_torch_stages = False
        self.profile_nsys_stages = False
        self.cuda_stage_events: dict = {}
        self._q_window: list[torch.Tensor] = []
        self._last_ids_dev: torch.Tensor | None = None
        self._last_ids_cpu: torch.Tensor | None = None
        self._last_prefill_ids: torch.Tensor | None = None
        self._last_verify_ids: torch.Tensor | None = None

    # -- state attributes ------------------------------------------------------
    @property
    def nblocks_filled(self) -> int:
        return self._core.nblocks_filled

    @nblocks_filled.setter
    def nblocks_filled(self, n: int) -> None:
        self._core.nblocks_filled = int(n)

    @property
    def valid_len(self) -> int:
        return self._core.valid_len

    @valid_len.setter
    def valid_len(self, n: int) -> None:
        self._core.valid_len = int(n)

    @property
    def prefill_len(self) -> int:
        return self._core.prefill_len

    @prefill_len.setter
    def prefill_len(self, n: int) -> None:
        self._core.prefill_len = int(n)

    @property
    def protected_blocks(self) -> set:
        return self._core.protected_blocks

    @protected_blocks.setter
    def protected_blocks(self, s) -> None:
        self._core.protected_blocks = set(s)

    def _ids_to_cpu(self, ids_dev):
        return None if ids_dev is None else ids_dev.to("cpu", torch.int64)

    @property
    def last_block_ids(self) -> torch.Tensor | None:
        """Selected ids of the last step as a CPU int64 tensor (copied on first read)."""
        if self._last_ids_cpu is None and self._last_ids_dev is not None:
            self._last_ids_cpu = self._ids_to_cpu(self._last_ids_dev)
        return self._last_ids_cpu

    @property
    def last_prefill_block_ids(self) -> torch.Tensor | None:
        return self._last_prefill_ids

    @property
    def last_verify_block_ids(self) -> torch.Tensor | None:
        return self._last_verify_ids

    def _set_last_ids(self, ids_dev: torch.Tensor) -> None:
        self._last_ids_dev = ids_dev
        self._last_ids_cpu = None

    def reset(self) -> None:
        """New sequence; buffers (and their contents) are kept (m12_runtime.py:322-349)."""
        self._core.reset()
        self._last_ids_dev = self._last_ids_cpu = None
        self._last_prefill_ids = self._last_verify_ids = None
        self.timings.clear()
        self.last_prefill_query_summaries = 0
        self.prefill_cpu_gather_ms = 0.0
        self.cuda_stage_events.clear()
        self.ids_history.clear()
        self.q_history.clear()
        self._q_window.clear()
        self._clear_selector_graph()
        self.selector_graph_setup_ms = 0.0
        self.selector_graph_builds = 0

    def reserve_blocks(self, nblocks: int) -> None:
        """The HBM history is allocated up front for max_model_len; only validate."""
        if nblocks > self.max_blocks:
            raise ValueError(f"{nblocks} blocks exceed max_model_len ({self.max_blocks} blocks)")

    # -- stage profiling (m12_runtime.py:1130-1136, :1155-1162) ---------------------
    def _profile_range(self, name: str):
        """A named profiler range when enabled: torch profiler (profile_torch_stages)
        or an NVTX / roctx range (profile_nsys_stages)."""
        if self.profile_torch_stages:
            return torch.profiler.record_function(f"m12.{name}")
        if self.profile_nsys_stages:
            return torch.cuda.nvtx.range(f"m12.{name}.layer{self.layer_id}")
        return nullcontext()

    def _event_pair(self, name: str):
        """With profile_cuda_stages: a timing-event pair stored under `name` in
        cuda_stage_events, its start recorded now on the current stream."""
        if not self.profile_cuda_stages:
            return None
        pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        self.cuda_stage_events[name] = pair
        pair[0].record()
        return pair

    @staticmethod
    def _event_end(pair) -> None:
        if pair is not None:
            pair[1].record()

    # -- caller overrides of the selector -----------------------------------------
    def _select_override(self):
        """An instance-level ``_gpu_select`` (the reference's tests force block ids
        by assigning one, tests/test_m14_prefill_layout.py:76), else None."""
        return self.__dict__.get("_gpu_select")

    def _ids_from_override(self, result) -> torch.Tensor:
        """Block ids an override returned, as a flat CPU int64 tensor.  Every id
        must name a filled history block: the kernels read blocks in place, so an
        id past the filled history (or negative) is refused here rather than
        attended as unwritten memory or skipped."""
        ids = result[0] if isinstance(result, tuple) else result
        ids = torch.as_tensor(ids).to("cpu", torch.int64).flatten()
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self.nblocks_filled):
            raise ValueError(f"_gpu_select override returned block ids outside [0, {self.nblocks_filled}) "
                             f"(min {int(ids.min())}, max {int(ids.max())})")
        return ids

    # -- exact attention over caller-packed K/V (m12_runtime.py:845-896) -------------
    def _fused_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, hist_len: int,
                         sink_len: int, causal_from: int, attn_mask: torch.Tensor | None = None) -> torch.Tensor:
        """q [Tq, Hq, D], k / v [S, Hkv, D] bf16 on the device -> [Tq, Hq, D] bf16.

        Query t sees key j iff j < causal_from + t + 1 (keys before causal_from
        are fully visible; causal_from >= S is the unmasked decode fast path),
        and, with attn_mask [Tq, S] (True = disallowed), only where the mask is
        False.  hist_len / sink_len describe the packing and do not change the
        result (as in the reference).  Runs on nkv_attend_packed: the few-query
        kernel (fp32 P.V) when Tq * G <= 16, else the matrix-core kernel (P
        rounded to bf16 for P.V, as flash-attention does)."""
        cfg = self.cfg
        if q.ndim != 3 or tuple(q.shape[1:]) != (cfg.num_heads, cfg.head_dim):
            raise ValueError(f"q must be [Tq, {cfg.num_heads}, {cfg.head_dim}] (got {tuple(q.shape)})")
        if k.ndim != 3 or tuple(k.shape[1:]) != (cfg.num_kv_heads, cfg.head_dim) or k.shape != v.shape:
            raise ValueError(f"k and v must be [S, {cfg.num_kv_heads}, {cfg.head_dim}] "
                             f"(got {tuple(k.shape)}, {tuple(v.shape)})")
        if min(hist_len, sink_len, causal_from) < 0:
            raise ValueError("hist_len, sink_len and causal_from must be >= 0")
        q = self._as_bf16(q, "q")
        k = self._as_bf16(k, "k")
        v = self._as_bf16(v, "v")
        return packed_attention(q, k, v, causal_from, cfg.scale, attn_mask)

    def _prefill_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           causal_from: int) -> torch.Tensor:
        """Packed later-chunk attention with the configured backend
        (m12_runtime.py:809-839).  "torch" is _fused_attention's masked path;
        "flash" is flash-attention's bottom-right causal alignment over the
        same keys, the same mask, so both run the same kernel here."""
        self._check_prefill_backend()
        return self._fused_attention(q, k, v, hist_len=causal_from, sink_len=0, causal_from=causal_from)

    def _check_prefill_backend(self) -> None:
        backend = self.cfg.prefill_attention_backend
        if backend not in ("torch", "flash"):
            raise ValueError(f"unknown prefill attention backend: {backend!r}")

    # -- input checks ------------------------------------------------------------
    def _as_bf16(self, t: torch.Tensor, name: str) -> torch.Tensor:
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
        return t.contiguous()

    # -- representatives / store -------------------------------------------------
    def _build_reps_gpu(self, k_blocks: torch.Tensor, start: int, nblocks: int) -> None:
        """k_blocks [N, B, Hkv, D] -> reps_gpu[:, start:start+N] (m12_runtime.py:354-395)."""
        kb = self._as_bf16(k_blocks[:nblocks], "k_blocks")
        n, b, hkv, d = kb.shape
        self._reps_changed()
        self.store.build_reps(self.store_layer, kb.reshape(1, n * b, hkv, d), start)

    def _store_kv(self, k: torch.Tensor, v: torch.Tensor) -> None:
        self._reps_changed()
        self._core.store_kv(self._as_bf16(k, "k").unsqueeze(0), self._as_bf16(v, "v").unsqueeze(0))

    def _reps_changed(self) -> None:
        """Representatives are about to be rebuilt: a captured selector graph is
        dropped (m12_runtime.py:362-363)."""
        self._clear_selector_graph()
        self._reps_version += 1

    def prefill_first(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> dict:
        """Store the first chunk; its dense attention is the caller's (m12_runtime.py:518-523)."""
        assert self.prefill_len == 0, "prefill_first called after history exists"
        with self._profile_range("prefill_first_store_kv"):
            self._store_kv(k, v)
        return {"nblocks": self.nblocks_filled, "valid_len": self.valid_len}

    def dense_prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      scale: float | None = None) -> torch.Tensor:
        """Causal attention of the first chunk within itself, on this library's kernels.

        The reference runs it through flash_attn_varlen_func(causal=True)
        before prefill_first (nanovllm/layers/attention.py:79-85); here it is
        the chunk path with nothing stored yet (no history, sink or recent).
        Call it before prefill_first.  q [T, Hq, D], k/v [T, Hkv, D] bf16 ->
        [T, Hq, D] bf16."""
        assert self.prefill_len == 0 and self.valid_len == 0, "dense_prefill is for the first chunk"
        q = self._as_bf16(q, "q")
        k = self._as_bf16(k, "k")
        v = self._as_bf16(v, "v")
        no_ids = self._core._buf("no_ids", 1, torch.int32)
        out, _, _ = self._core.chunk_attend(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                            no_ids, 1, 0, scale=scale)
        return out[0]

    # -- selection -------------------------------------------------------------------
    def _select_dev(self, q3: torch.Tensor, requested: int, order: int, use_graph: bool = False):
        if use_graph:
            return self._graph_select(q3, requested, order)
        ids, vals, k = self._core.select(q3.unsqueeze(0), requested, order=order)
        return ids, vals, k

    # -- selector graph (m12_runtime.py:294-299, :901-957) -------------------------
    def _clear_selector_graph(self) -> None:
        self._selector_graph = None
        self._selector_graph_key = None
        self._selector_graph_q = None
        self._selector_graph_outputs = None
        self._selector_graph_keep = None

    def _graph_select(self, q3: torch.Tensor, requested: int, order: int):
        """The score + top-k launches captured once in a HIP graph and replayed.

        A capture serves one (history length, budget, protected set within the
        history, query shape, id order, representatives' storage and version);
        any change captures anew (one graph per runtime, as m12_runtime.py:
        916-957 keeps), counted in selector_graph_builds with its set-up time
        in selector_graph_setup_ms.  The representatives are read through the
        same pointer on every replay, so in-place edits are seen.  Returns the
        graph's own (ids, vals) buffers, rewritten by the next replay, and k.
        Same kernels and results as the eager selection (neither clears memory
        with a memset: the top-k leaves the score keys zero)."""
        nb = self.nblocks_filled
        if nb <= 0:
            raise ValueError("selection needs at least one history block")
        prot_ids = tuple(sorted(p for p in self.protected_blocks if 0 <= p < nb))
        key = (nb, int(requested), prot_ids, tuple(q3.shape), q3.dtype, q3.device, int(order),
               self.reps_gpu.data_ptr(), self._reps_version)
        if key != self._selector_graph_key:
            self._clear_selector_graph()
            started = perf_counter()
            dev = q3.device
            static_q = q3.detach().clone()
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                # the eager run allocates every workspace (and the protected
                # list) the capture then records, so nothing is allocated
                # inside it
                self._core.select(static_q.unsqueeze(0), requested, order=order, ws="/graph")
            side.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                graph.capture_begin()
                try:
                    ids, vals, k = self._core.select(static_q.unsqueeze(0), requested, order=order,
                                                     ws="/graph")
                finally:
                    graph.capture_end()
            torch.cuda.current_stream(dev).wait_stream(side)
            self._selector_graph = graph
            self._selector_graph_q = static_q
            self._selector_graph_outputs = (ids, vals, k)
            # the buffers the graph reads and writes stay alive with it
            self._selector_graph_keep = (self._core.protected_dev()[0], dict(self._core._ws))
            self._selector_graph_key = key
            self.selector_graph_setup_ms += (perf_counter() - started) * 1000.0
            self.selector_graph_builds += 1
        self._selector_graph_q.copy_(q3)
        self._selector_graph.replay()
        return self._selector_graph_outputs

    def _gpu_select(self, q: torch.Tensor, *, dynamic: bool = False, budget: int | None = None,
                    use_graph: bool = False, use_static_mask: bool = False,
                    use_relative: bool = False):
        """Block scores + Top-K; returns (block_ids_cpu [K] int64, info).

        Reference: m12_runtime.py:959-1055.  With use_graph and
        cfg.selector_cuda_graph the two launches (score, Top-K) replay from a
        captured HIP graph (_graph_select); the static-mask option selects the
        same launches (the protected list is cached on the device either way).
        """
        cfg = self.cfg
        if q.ndim == 2:
            q = q.unsqueeze(0)
        assert q.ndim == 3 and q.shape[1:] == (cfg.num_heads, cfg.head_dim)
        q = self._as_bf16(q, "q")
        if use_relative and (use_graph and cfg.selector_cuda_graph):
            raise ValueError("relative-threshold selection requires the flat GPU path")
        requested_k = cfg.top_k_blocks if budget is None else budget
        t_enq = perf_counter()
        ids_cpu, vals_cpu, k = self._select_host(q, requested_k, use_relative,
                                                 use_graph=use_graph and cfg.selector_cuda_graph)
        t_d2h = perf_counter()
        chosen = k
        if dynamic and cfg.dynamic_top_k and k == requested_k:
            chosen = dynamic_top_k_from_scores(vals_cpu, requested_k, cfg.dynamic_top_k_mass)
        if chosen < k:
            ids_cpu = ids_cpu[:chosen]
        d2h_ms = (perf_counter() - t_d2h) * 1000.0
        return ids_cpu, {
            "d2h_ms": d2h_ms,
            "enqueue_ms": (t_d2h - t_enq) * 1000.0,
            "n_selected": chosen,
            "n_candidates": k,
            "n_query_summaries": q.shape[0],
        }

    def _select_host(self, q: torch.Tensor, requested_k: int, use_relative: bool, use_graph: bool = False):
        """Selected ids and scores on the host (score-desc order)."""
        cfg = self.cfg
        if not use_relative:
            ids, vals, k = self._select_dev(q, requested_k, _lib.NKV_ORDER_SCORE_DESC, use_graph=use_graph)
            return ids[0, 0, :k].to("cpu", torch.int64), vals[0, 0, :k].cpu(), k
        # relative threshold (m12_runtime.py:1015-1031): keep candidates within
        # ln(a)/scale of the best among the top `cap`, or top-k in union mode.
        a = cfg.decode_relative_a
        assert a is not None and 0.0 < a < 1.0
        nb = self.nblocks_filled
        n_prot = len([p for p in self.protected_blocks if 0 <= p < nb])
        avail = nb - n_prot
        k = min(requested_k, max(1, avail))
        cap = min(cfg.decode_relative_max_blocks, max(1, avail))
        req = max(cap, k)
        ids, vals, keff = self._select_dev(q, req, _lib.NKV_ORDER_SCORE_DESC)
        order = ids[0, 0, :keff].to("cpu", torch.int64)
        scores = vals[0, 0, :keff].cpu()
        threshold = float(scores[0]) + math.log(a) / cfg.scale
        cand, cs = order[:cap], scores[:cap]
        above = cs >= threshold
        if cfg.decode_relative_union:
            pos = torch.arange(cand.numel()) < k
            keep = above | pos
        else:
            keep = above
        if not bool(keep.any()):
            return order[:k], scores[:k], k
        return cand[keep], cs[keep], int(keep.sum())

    def _gpu_select_per_query(self, q: torch.Tensor, k: int):
        """Per-query Top-K, union (sorted) and allowed mask (m12_runtime.py:1057-1087)."""
        cfg = self.cfg
        if q.ndim == 2:
            q = q.unsqueeze(0)
        q = self._as_bf16(q, "q")
        tq = q.shape[0]
        if tq > 16:
            raise ValueError("per-query selection supports at most 16 queries")
        ids, _, kk = self._core.select(q.unsqueeze(0), int(k), per_query=True)
        top = ids[0, :, :kk].to("cpu", torch.int64)                 # [Tq, kk]
        union = torch.unique(top.flatten())
        pos = torch.searchsorted(union, top.flatten()).reshape(tq, kk)
        allowed = torch.zeros(tq, union.numel(), dtype=torch.bool)
        allowed.scatter_(1, pos, True)
        return union, allowed.to(q.device)

    def diagnose_target_margin(self, q: torch.Tensor, target_block: int) -> dict:
        """Score margin of one block under the decode selector (m12_runtime.py:1089-1128)."""
        cfg = self.cfg
        if q.ndim == 2:
            q = q.unsqueeze(0)
        q = self._as_bf16(q, "q")
        ids, _, k = self._select_dev(q, cfg.top_k_blocks, _lib.NKV_ORDER_SCORE_DESC)
        scores = self._core._last_scores[0, 0].cpu().clone()
        nb = self.nblocks_filled
        prot = [p for p in self.protected_blocks if 0 <= p < nb]
        if prot:
            scores[torch.tensor(sorted(prot))] = float("-inf")
        order = sorted(range(nb), key=lambda i: (-float(scores[i]), i))
        rank = order.index(int(target_block))
        return {
            "target_score": float(scores[int(target_block)]),
            "cutoff": float(scores[order[k - 1]]),
            "rank": rank,
            "nblocks": nb,
            "in_topk": rank < k,
        }

    # -- decode (m12_runtime.py:1141-1346) ---------------------------------------------
    def decode(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, device=None) -> torch.Tensor:
        """One decode step.  q [1, Hq, D], k/v [1, Hkv, D] bf16 -> o [1, Hq, D] bf16."""
        cfg = self.cfg
        assert q.shape[0] == 1 and k.shape[0] == 1
        q = self._as_bf16(q, "q")
        k = self._as_bf16(k, "k")
        v = self._as_bf16(v, "v")
        if self.record_q:
            self.q_history.append(q[0].detach().cpu().clone())
        t0 = perf_counter()
        if cfg.decode_query_window > 1:
            self._q_window.append(q[0].detach().clone())
            while len(self._q_window) > cfg.decode_query_window:
                self._q_window.pop(0)
            if len(self._q_window) == 1:
                q_route = self._q_window[0].unsqueeze(0)
            else:
                q_route = prefill_query_summaries(torch.stack(self._q_window, dim=0), 1)
        else:
            q_route = q
        requested = cfg.top_k_blocks if cfg.decode_top_k_blocks is None else cfg.decode_top_k_blocks
        override = self._select_override()
        host_rule = cfg.decode_relative_a is not None or cfg.dynamic_top_k or override is not None
        if (self.device_ring and self.device_ring_ready() and override is None
                and not self.profile_cuda_stages and not cfg.selector_cuda_graph):
            return self._decode_ring(q, k, v, requested, t0)
        # the recent append runs inside the attention launch (the new token is
        # written to the ring slot it frees), so its event pair spans nothing
        ev = self._event_pair("recent")
        self._event_end(ev)
        ev = self._event_pair("selector")
        with self._profile_range("selector"):
            if override is not None:
                ids_cpu = self._ids_from_override(override(
                    q_route[0], dynamic=cfg.dynamic_top_k, budget=cfg.decode_top_k_blocks,
                    use_graph=cfg.selector_cuda_graph, use_static_mask=cfg.selector_static_mask,
                    use_relative=cfg.decode_relative_a is not None))
            elif host_rule:
                ids_cpu, info = self._gpu_select(q_route, dynamic=cfg.dynamic_top_k, budget=requested,
                                                 use_graph=cfg.selector_cuda_graph,
                                                 use_static_mask=cfg.selector_static_mask,
                                                 use_relative=cfg.decode_relative_a is not None)
            if host_rule:
                if cfg.gather_sort and ids_cpu.numel() > 1:
                    ids_cpu = ids_cpu.sort().values
                n_hist = ids_cpu.numel()
                ids_dev = ids_cpu.to(torch.int32).to(self.store.device).view(1, 1, n_hist)
                stride = n_hist
            else:
                order = _lib.NKV_ORDER_ID_ASC if cfg.gather_sort else _lib.NKV_ORDER_SCORE_DESC
                ids_dev, _, n_hist = self._select_dev(q_route, requested, order,
                                                      use_graph=cfg.selector_cuda_graph)
                stride = ids_dev.shape[-1]
        self._event_end(ev)
        selector_ms = (perf_counter() - t0) * 1000.0
        # the selected blocks are read in place: no gather, no pack
        ev = self._event_pair("h2d_pack")
        self._event_end(ev)
        t_a = perf_counter()
        ev = self._event_pair("packed_attention")
        with self._profile_range("packed_attention"):
            out, sink_len, rec_len = self._core.decode_attend(
                q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), ids_dev, stride, n_hist)
        self._event_end(ev)
        attn_ms = (perf_counter() - t_a) * 1000.0
        self._set_last_ids(ids_dev[0, 0, :n_hist])
        if self.record_ids:
            self.ids_history.append(self.last_block_ids.tolist())
        sel_tokens = n_hist * cfg.block_size
        self.timings = {
            "selector_ms": selector_ms,
            "selector_enqueue_ms": selector_ms,
            "d2h_ms": 0.0,
            "cpu_gather_ms": 0.0,
            "h2d_pack_ms": 0.0,
            "h2d_event_spans_cpu_gather": False,
            "recent_ms": 0.0,
            "packed_attn_ms": attn_ms,
            "selected_tokens": sel_tokens,
            "total_attend_tokens": sel_tokens + sink_len + rec_len,
        }
        o = out[0]
        if cfg.check_finite_outputs and not bool(torch.isfinite(o).all()):
            raise RuntimeError("M12 sparse decode output is non-finite")
        return o

    # -- replaying a captured device-ring decode step -----------------------------
    def device_ring_ready(self) -> bool:
        """Whether decode() would take the device-ring entry with device_ring set."""
        cfg = self.cfg
        return (cfg.decode_relative_a is None and not cfg.dynamic_top_k and not cfg.gather_sort
                and cfg.decode_query_window <= 1 and self._core.decode_ring_ready())

    def decode_state(self) -> tuple:
        """(ring start, valid length, device ring value): the host state a decode step moves."""
        c = self._core
        return c.ring_start, c.valid_len, c._ring_dev_pos

    def restore_decode_state(self, state: tuple) -> None:
        """Undo the host side of a decode step that was captured, not run."""
        c = self._core
        c.ring_start, c.valid_len, c._ring_dev_pos = state

    def ring_replayed(self) -> None:
        """Host side of one replay of a captured device-ring decode step: the
        ring and length move as in decode(); the ids are re-read on demand."""
        self._core.advance_ring()
        self._last_ids_cpu = None

    def _decode_ring(self, q, k, v, requested: int, t0: float) -> torch.Tensor:
        """decode() through the device-ring entry (same kernels and results)."""
        cfg = self.cfg
        out, ids_dev, n_hist, w = self._core.decode_ring(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                                         requested)
        self._set_last_ids(ids_dev[0, 0, :n_hist])
        if self.record_ids:
            self.ids_history.append(self.last_block_ids.tolist())
        ms = (perf_counter() - t0) * 1000.0
        sel_tokens = n_hist * cfg.block_size
        self.timings = {
            "selector_ms": 0.0, "selector_enqueue_ms": 0.0, "d2h_ms": 0.0, "cpu_gather_ms": 0.0,
            "h2d_pack_ms": 0.0, "h2d_event_spans_cpu_gather": False, "recent_ms": 0.0,
            "packed_attn_ms": ms, "selected_tokens": sel_tokens,
            "total_attend_tokens": sel_tokens + w["sink_len"] + w["rec_len"] + 1,
        }
        o = out[0]
        if cfg.check_finite_outputs and not bool(torch.isfinite(o).all()):
            raise RuntimeError("M12 sparse decode output is non-finite")
        return o

    # -- chunked prefill (m12_runtime.py:528-651) ---------------------------------------
    def prefill_chunk(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, device=None) -> torch.Tensor:
        """Later prefill chunk: attention over [selected | sink | prev recent | chunk]."""
        cfg = self.cfg
        assert self.prefill_len > 0, "prefill_chunk requires prior history"
        assert not (self.quant_history and cfg.prefill_adapter is not None), \
            "quant_history is incompatible with the segmented prefill adapter"
        self._check_prefill_backend()
        q = self._as_bf16(q, "q")
        k = self._as_bf16(k, "k")
        v = self._as_bf16(v, "v")
        with self._profile_range("prefill_selector"):
            q_summary = prefill_query_summaries(q, cfg.prefill_query_segments)
            self.last_prefill_query_summaries = q_summary.shape[0]
            requested = cfg.top_k_blocks if cfg.prefill_top_k_blocks is None else cfg.prefill_top_k_blocks
            override = self._select_override()
            if cfg.prefill_selection == "tile" and override is None and cfg.prefill_adapter is None:
                return self._prefill_chunk_tiled(q, k, v, requested)
            if override is not None:
                res = override(q_summary) if cfg.prefill_top_k_blocks is None else \
                    override(q_summary, budget=cfg.prefill_top_k_blocks)
                ids_cpu = self._ids_from_override(res)
                if cfg.gather_sort and ids_cpu.numel() > 1:
                    ids_cpu = ids_cpu.sort().values
                n_hist = ids_cpu.numel()
                ids_dev = ids_cpu.to(torch.int32).to(self.store.device).view(1, 1, n_hist)
            else:
                order = _lib.NKV_ORDER_ID_ASC if cfg.gather_sort else _lib.NKV_ORDER_SCORE_DESC
                ids_dev, _, n_hist = self._select_dev(q_summary, requested, order)
                ids_cpu = None
        if cfg.prefill_adapter is not None:
            out = self._adapter_attention(cfg.prefill_adapter, q, k, v, ids_dev[0, 0, :n_hist])
        else:
            with self._profile_range("prefill_attention"):
                out = self._core.chunk_attend(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                              ids_dev, ids_dev.shape[-1], n_hist)[0][0]
        if ids_cpu is None:
            ids_cpu = ids_dev[0, 0, :n_hist].to("cpu", torch.int64)
        with self._profile_range("prefill_store_kv"):
            self._store_kv(k, v)
        self._last_prefill_ids = ids_cpu.clone()
        self._last_ids_dev = None
        self._last_ids_cpu = ids_cpu
        return out

    def _prefill_chunk_tiled(self, q, k, v, requested: int) -> torch.Tensor:
        """prefill_chunk with prefill_selection="tile": one Top-K per tile of
        prefill_selection_tile queries (from the tile's query mean); each
        tile's queries attend [its blocks | sink | previous recent | chunk
        (causal)].  last_prefill_block_ids is then [ntiles, K]."""
        cfg = self.cfg
        tile = cfg.prefill_selection_tile
        order = _lib.NKV_ORDER_ID_ASC if cfg.gather_sort else _lib.NKV_ORDER_SCORE_DESC
        ids, n_hist = self._core.select_tiles(q.unsqueeze(0), requested, tile, order)
        self.last_prefill_query_summaries = ids.shape[1]
        with self._profile_range("prefill_attention"):
            out = self._core.chunk_attend_tiled(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), ids, tile,
                                                n_hist)[0][0]
        ids_cpu = ids[0, :, :n_hist].to("cpu", torch.int64)
        with self._profile_range("prefill_store_kv"):
            self._store_kv(k, v)
        self._last_prefill_ids = ids_cpu.clone()
        self._last_ids_dev = None
        self._last_ids_cpu = ids_cpu
        return out

    def _adapter_attention(self, adapter, q, k, v, ids_dev) -> torch.Tensor:
        """The segmented-prefill adapter contract (segmented_prefill_adapter.py:95-147,
        m12_runtime.py:596-611, :633-636): adapter.prepare(q, selected_k,
        selected_v, (sink_k, sink_v), (recent_k, recent_v), (k, v)) then
        adapter.attend(invocation) -> o.  Every segment is token-major
        [tokens, Hkv, D]: the selected blocks gathered from the history (device
        tensors; pinned host tensors with history_tier="host"), the sink, the
        previous recent window in logical order, the chunk."""
        cfg = self.cfg
        st, L = self.store, self.store_layer
        R, D, hkv = cfg.recent_tokens, cfg.head_dim, cfg.num_kv_heads
        with self._profile_range("prefill_h2d_pack"):
            ids = ids_dev.to(torch.int64)
            if st.history_tier == "host":
                ids = ids.cpu()
            # contiguous before pinning: pin_memory keeps a view's strides, and
            # a later .contiguous() would make a pageable copy
            sel_k = st.hist_k[L][:, ids].permute(1, 2, 0, 3).reshape(-1, hkv, D).contiguous()
            sel_v = st.hist_v[L][:, ids].permute(1, 2, 0, 3).reshape(-1, hkv, D).contiguous()
            if st.history_tier == "host":
                sel_k, sel_v = sel_k.pin_memory(), sel_v.pin_memory()
            sink_len = min(cfg.sink_tokens, self.valid_len)
            _, off, ln = prefill_recent_slice(self.valid_len, cfg.sink_tokens, R)
            slots = (torch.arange(off, off + ln, device=st.device) + self._core.ring_start) % R
            sink = (st.sink_k[L][:, :sink_len].permute(1, 0, 2).contiguous(),
                    st.sink_v[L][:, :sink_len].permute(1, 0, 2).contiguous())
            recent = (st.recent_k[L][:, slots].permute(1, 0, 2).contiguous(),
                      st.recent_v[L][:, slots].permute(1, 0, 2).contiguous())
            invocation = adapter.prepare(q, sel_k, sel_v, sink, recent, (k, v))
        with self._profile_range("prefill_attention"):
            return adapter.attend(invocation)

    # -- speculative verify (m12_runtime.py:656-807) -------------------------------------
    def verify_tokens(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, device=None) -> torch.Tensor:
        """One verification pass over Tq new tokens; commit or roll back afterwards."""
        cfg = self.cfg
        tq = k.shape[0]
        assert tq >= 1, "verify needs at least one token"
        assert self.prefill_len > 0, "verify requires a complete prefill"
        assert not (self.quant_history and cfg.prefill_adapter is not None), \
            "quant_history is incompatible with the segmented prefill adapter"
        q = self._as_bf16(q, "q")
        k = self._as_bf16(k, "k")
        v = self._as_bf16(v, "v")
        if not self.verify_lossless:   # the shared selection's attention is _prefill_attention's
            self._check_prefill_backend()
        t0 = perf_counter()
        allowed_dev = None
        override = self._select_override()
        with self._profile_range("verify_selector"):
            if self.verify_lossless:
                union, allowed = self._gpu_select_per_query(q, cfg.top_k_blocks)
                union = torch.as_tensor(union).to("cpu", torch.int64).flatten()
                ids_dev = union.to(torch.int32).to(self.store.device).view(1, 1, -1)
                n_hist = union.numel()
                allowed_dev = torch.as_tensor(allowed).to(self.store.device, torch.uint8).contiguous()
                ids_cpu = union
            elif override is not None:
                ids_cpu = self._ids_from_override(override(q))
                n_hist = ids_cpu.numel()
                ids_dev = ids_cpu.to(torch.int32).to(self.store.device).view(1, 1, n_hist)
            else:
                ids_dev, _, n_hist = self._select_dev(q, cfg.top_k_blocks, _lib.NKV_ORDER_SCORE_DESC)
                ids_cpu = None
        t_sel = perf_counter()
        with self._profile_range("verify_attention"):
            out, _, _ = self._core.chunk_attend(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                                ids_dev, ids_dev.shape[-1], n_hist, allowed_dev)
        t_attn = perf_counter()
        if ids_cpu is None:
            ids_cpu = ids_dev[0, 0, :n_hist].to("cpu", torch.int64)
        self.last_verify_timings = {
            "selector_ms": (t_sel - t0) * 1000.0,
            "gather_ms": 0.0,
            "pack_ms": 0.0,
            "attention_ms": (t_attn - t_sel) * 1000.0,
            "tokens": int(tq),
            "blocks": int(n_hist),
        }
        self._core.pending = (k.unsqueeze(0), v.unsqueeze(0))
        self._last_verify_ids = ids_cpu.clone()
        self._last_ids_dev = None
        self._last_ids_cpu = ids_cpu
        return out[0]

    def commit_verified(self, n: int) -> None:
        """Append the first n pending verified tokens to the recent window."""
        self._core.commit(n)

    def rollback_verified(self) -> None:
        """Discard a verification pass without committing anything."""
        self._core.pending = None

    @property
    def _pending_k(self):
        return None if self._core.pending is None else self._core.pending[0][0]

    @property
    def _pending_v(self):
        return None if self._core.pending is None else self._core.pending[1][0]


# ---------------------------------------------------------------------------
# All layers of a model at once
# ---------------------------------------------------------------------------


class M12ModelRuntime:
    """The sparse layer-step for every attention layer of a model, batched.

    One store holds all layers; each stage is one kernel launch over all
    layers (grid dimension = layer).  Inputs carry a leading layer dimension:
    q [L, T, Hq, D], k/v [L, T, Hkv, D].  Semantics per layer are exactly
    those of M12LayerRuntime (all layers share the sequence bookkeeping).

    decode() is one native call (nkv_decode_step): selection then attention
    for every layer, the layers split into `layer_streams` contiguous ranges
    on as many streams (the caller's current stream first).  The layers are
    independent and each range makes the launches a one-range call would, so
    the result does not depend on layer_streams.  More ranges let one range's
    launch-bound top-k and merge kernels overlap another's bandwidth-bound
    kernels, but each step then pays two cross-stream joins; on the 36-layer
    32K step one range is faster (128 vs 135 us), hence the default.
    """

    def __init__(self, num_layers: int, cfg: M12Config, device=None, layer_streams: int = 1):
        _check_hip_shapes(cfg)
        self.cfg = cfg
        self.num_layers = num_layers
        B = cfg.block_size
        self.max_blocks = (cfg.max_model_len + B - 1) // B
        self.store = SparseKVStore(
            num_layers, num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads,
            head_dim=cfg.head_dim, block_size=B, r=cfg.r, cap_blocks=self.max_blocks,
            sink_tokens=cfg.sink_tokens, recent_tokens=cfg.recent_tokens,
            kv_format=cfg.kv_format, device=device,
                history_tier=cfg.history_tier)
        self.core = _SparseCore(cfg, self.store, 0, num_layers)
        self.last_ids_dev: torch.Tensor | None = None
        self.last_n_selected = 0
        if layer_streams < 1:
            raise ValueError("layer_streams must be >= 1")
        self.layer_streams = min(layer_streams, num_layers)
        self._side_streams: list = []   # created on the first decode (default priority)
        self.last_union_dev: torch.Tensor | None = None
        self.last_union_count_dev: torch.Tensor | None = None

    @property
    def valid_len(self) -> int:
        return self.core.valid_len

    @property
    def nblocks_filled(self) -> int:
        return self.core.nblocks_filled

    def reset(self) -> None:
        self.core.reset()

    def prefill(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Store a prefill chunk for every layer: k, v [L, T, Hkv, D] bf16."""
        self.core.store_kv(k, v)

    def prefill_chunk(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """A later prefill chunk for every layer (M12LayerRuntime.prefill_chunk per layer).

        q [L, T, Hq, D], k/v [L, T, Hkv, D] -> o [L, T, Hq, D]: query summaries,
        selection, attention over [selected | sink | previous recent | chunk],
        then the chunk is stored (m12_runtime.py:528-651).
        """
        cfg = self.cfg
        if self.core.prefill_len <= 0:
            raise ValueError("prefill_chunk requires prior history")
        req = cfg.top_k_blocks if cfg.prefill_top_k_blocks is None else cfg.prefill_top_k_blocks
        order = _lib.NKV_ORDER_ID_ASC if cfg.gather_sort else _lib.NKV_ORDER_SCORE_DESC
        if cfg.prefill_selection == "tile":
            ids, n = self.core.select_tiles(q.contiguous(), req, cfg.prefill_selection_tile, order)
            out, _, _ = self.core.chunk_attend_tiled(q, k, v, ids, cfg.prefill_selection_tile, n)
        else:
            qs = query_summaries(q.contiguous(), cfg.prefill_query_segments)
            ids, _, n = self.core.select(qs, req, order=order)
            out, _, _ = self.core.chunk_attend(q, k, v, ids, ids.shape[-1], n)
        self.core.store_kv(k, v)
        self.last_ids_dev = ids
        self.last_n_selected = n
        return out

    def verify(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
               lossless: bool = False) -> torch.Tensor:
        """One speculative verification pass for every layer (M12LayerRuntime.verify_tokens,
        m12_runtime.py:656-758): q [L, Tq, Hq, D], k/v [L, Tq, Hkv, D] -> o [L, Tq, Hq, D].

        shared: one selection from the Tq queries (max-reduced scores).  lossless:
        a Top-K per query, their union and the per-query mask built on the device
        (nkv_select_union, no host round trip), so query t attends only its own
        blocks.  The Tq tokens are attended causally and held pending:
        commit_verified(n) appends the first n to the recent window,
        rollback_verified() drops them."""
        cfg, core = self.cfg, self.core
        if core.prefill_len <= 0:
            raise ValueError("verify requires a complete prefill")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        L, tq = q.shape[0], q.shape[1]
        req = cfg.top_k_blocks
        if lossless:
            if tq > 16:
                raise ValueError("per-query selection supports at most 16 queries")
            union, count, allowed, umax = core.select_per_query_union(q, req)
            out, _, _ = core.chunk_attend(q, k, v, union, umax, umax, allowed, allowed_stride=tq * umax)
            self.last_union_dev, self.last_union_count_dev = union, count
        else:
            ids, _, n = core.select(q, req)
            out, _, _ = core.chunk_attend(q, k, v, ids, ids.shape[-1], n)
            self.last_union_dev, self.last_union_count_dev = ids[:, 0, :n], None
        core.pending = (k, v)
        return out

    def commit_verified(self, n: int) -> None:
        """Append the first n pending verified tokens of every layer to the recent window."""
        self.core.commit(n)

    def rollback_verified(self) -> None:
        """Discard the pending verification pass."""
        self.core.pending = None

    def select(self, q: torch.Tensor, budget: int | None = None):
        """Decode selection for every layer: q [L, 1, Hq, D] -> (ids [L, 1, K], vals, k)."""
        cfg = self.cfg
        req = budget or (cfg.top_k_blocks if cfg.decode_top_k_blocks is None else cfg.decode_top_k_blocks)
        return self.core.select(q, req)

    def decode(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """One decode step for every layer: q [L, 1, Hq, D], k/v [L, 1, Hkv, D] -> o [L, 1, Hq, D]."""
        cfg, core = self.cfg, self.core
        nb = core.nblocks_filled
        if nb <= 0:
            raise ValueError("selection needs at least one history block")
        L = self.num_layers
        if (q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16
                or tuple(q.shape) != (L, 1, cfg.num_heads, cfg.head_dim)
                or tuple(k.shape) != (L, 1, cfg.num_kv_heads, cfg.head_dim) or k.shape != v.shape
                or not (q.is_cuda and k.is_cuda and v.is_cuda)):
            raise ValueError(f"decode expects bf16 device tensors q [{L}, 1, {cfg.num_heads}, {cfg.head_dim}] "
                             f"and k, v [{L}, 1, {cfg.num_kv_heads}, {cfg.head_dim}]")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        w = core.decode_window()
        plan = self._step_plan(nb, w)
        out = torch.empty_like(q)
        ids = torch.empty(L, 1, plan["req"], dtype=torch.int32, device=q.device)
        _lib.check(self.store.lib.nkv_decode_step(
            self.store._desc_ref, 0, L, q.data_ptr(), k.data_ptr(), v.data_ptr(), nb, plan["prot_ptr"],
            plan["n_prot"], plan["req"], plan["n"], w["sink_len"], w["write_slot"], w["ring_base"], w["rec_lo"],
            w["rec_len"], plan["scale"], plan["splits"], plan["keys_ptr"], ids.data_ptr(), plan["part_ptr"],
            out.data_ptr(), plan["nstreams"], plan["streams"]), "decode_step")
        core.advance_decode()
        self.last_ids_dev = ids
        self.last_n_selected = plan["n"]
        return out

    def _step_plan(self, nb: int, w: dict) -> dict:
        """The decode step's launch arguments that only change with the history
        length, the protected set, the window shape and the current stream
        (workspaces, split count, effective budget, the stream list)."""
        cfg, core = self.cfg, self.core
        prot, n_prot = core.protected_dev()
        dev = self.store.device
        cur = current_stream_ptr(dev)
        key = (nb, core._prot_key, w["sink_len"], w["rec_len"] > 0, cur, cfg.top_k_blocks, cfg.decode_top_k_blocks,
               cfg.attend_splits, cfg.scale, self.layer_streams)
        plan = getattr(self, "_plan", None)
        if plan is not None and plan["key"] == key:
            return plan
        req = cfg.top_k_blocks if cfg.decode_top_k_blocks is None else cfg.decode_top_k_blocks
        L = self.num_layers
        if len(self._side_streams) < self.layer_streams - 1:
            self._side_streams = [torch.cuda.Stream(dev) for _ in range(self.layer_streams - 1)]
        streams = [cur] + [s.cuda_stream for s in self._side_streams[:self.layer_streams - 1]]
        n = core.effective_k(req)
        splits = core.decode_splits(n)
        keys = core._zeroed_keys(L * nb, "/step")
        part = core._buf("partial/step", self.store.decode_step_workspace_floats(L, splits, len(streams)),
                         torch.float32)
        plan = {"key": key, "req": req, "n": n, "splits": splits, "n_prot": n_prot, "scale": float(cfg.scale),
                "prot_ptr": prot.data_ptr(), "keys_ptr": keys.data_ptr(), "part_ptr": part.data_ptr(),
                "nstreams": len(streams), "streams": (ctypes.c_void_p * len(streams))(*streams),
                "_keep": (prot, keys, part)}
        self._plan = plan
        return plan
