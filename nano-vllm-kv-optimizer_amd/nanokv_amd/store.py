"""HBM-resident sparse KV store for a stack of attention layers.

The reference keeps the post-RoPE history on the host and copies the selected
blocks to the GPU every decode step (nanovllm/sparse/m12_runtime.py:185-246,
:1212-1311).  Here the whole history lives in HBM, head-major so that one
(KV head, block) is 16 KiB contiguous:

    hist_k / hist_v : [L, Hkv, cap, 64, 128]  bf16, or int8 + scales
    reps            : [L, Hkv, cap, r, 128]   bf16 (the reference's reps_gpu layout)
    sink_k / sink_v : [L, Hkv, S, 128]        bf16
    recent_k / _v   : [L, Hkv, R, 128]        bf16 ring (logical slot i at (ring_start + i) % R)

Every method enqueues HIP kernels on the current torch stream through the C
ABI of include/nanokv.h; none of them synchronises.

history_tier="host" keeps hist_k / hist_v (the bulk: 16 KiB per (block, KV
head) each) in pinned host memory instead, for histories larger than HBM,
as the reference always does.  Everything else stays in HBM, and the same
kernels read the selected blocks in place through the device mapping of the
pinned pages (nkv_host_device_pointer): the reference's per-step gather into
pinned staging and H2D copy (m12_runtime.py:1212-1311) has no counterpart.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

KV_FORMATS = {
    "bf16": _lib.NKV_KV_BF16,
    "int8": _lib.NKV_KV_INT8_CHANNEL,
    "int8_token": _lib.NKV_KV_INT8_TOKEN,
}

HEAD_DIM = 128
BLOCK_SIZE = 64


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_ptr(device=None) -> int:
    """Raw handle of the current stream of `device` (default: the current
    device), without building a torch Stream object on every launch."""
    if _raw_stream is not None:
        idx = None if device is None else torch.device(device).index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


def _stream():
    return ctypes.c_void_p(current_stream_ptr())


class SparseKVStore:
    """Device buffers of one model's sparse attention history (all layers)."""

    def __init__(self, num_layers: int, *, num_heads: int, num_kv_heads: int, head_dim: int,
                 block_size: int, r: int, cap_blocks: int, sink_tokens: int, recent_tokens: int,
                 kv_format: str = "bf16", device=None, history_tier: str = "hbm"):
        if head_dim != HEAD_DIM:
            raise ValueError(f"head_dim must be {HEAD_DIM} for the gfx950 kernels (got {head_dim})")
        if block_size != BLOCK_SIZE:
            raise ValueError(f"block_size must be {BLOCK_SIZE} for the gfx950 kernels (got {block_size})")
        if kv_format not in KV_FORMATS:
            raise ValueError(f"unknown kv_format {kv_format!r}")
        if history_tier not in ("hbm", "host"):
            raise ValueError(f"history_tier must be 'hbm' or 'host' (got {history_tier!r})")
        self.lib = _lib.load()
        dev = torch.device(device if device is not None else "cuda")
        L, H, S, R, B, D = num_layers, num_kv_heads, sink_tokens, recent_tokens, block_size, head_dim
        self.num_layers, self.num_heads, self.num_kv_heads = L, num_heads, num_kv_heads
        self.head_dim, self.block_size, self.r = D, B, r
        self.cap_blocks, self.sink_tokens, self.recent_tokens = cap_blocks, S, R
        self.kv_format = kv_format
        self.device = dev
        self.history_tier = history_tier
        hdt = torch.bfloat16 if kv_format == "bf16" else torch.int8
        if history_tier == "host":
            # new pinned allocations (the HIP runtime maps them for the device)
            self.hist_k = torch.zeros(L, H, cap_blocks, B, D, dtype=hdt, pin_memory=True)
            self.hist_v = torch.zeros(L, H, cap_blocks, B, D, dtype=hdt, pin_memory=True)
            with torch.cuda.device(dev):
                hist_k_addr = _lib.host_device_pointer(self.hist_k.data_ptr())
                hist_v_addr = _lib.host_device_pointer(self.hist_v.data_ptr())
        else:
            self.hist_k = torch.zeros(L, H, cap_blocks, B, D, dtype=hdt, device=dev)
            self.hist_v = torch.zeros_like(self.hist_k)
            hist_k_addr, hist_v_addr = self.hist_k.data_ptr(), self.hist_v.data_ptr()
        self.reps = torch.zeros(L, H, cap_blocks, r, D, dtype=torch.bfloat16, device=dev)
        self.sink_k = torch.zeros(L, H, max(S, 1), D, dtype=torch.bfloat16, device=dev)
        self.sink_v = torch.zeros_like(self.sink_k)
        self.recent_k = torch.zeros(L, H, R, D, dtype=torch.bfloat16, device=dev)
        self.recent_v = torch.zeros_like(self.recent_k)
        self.k_scale = self.v_scale = self.k_tscale = self.v_tscale = None
        if kv_format == "int8":
            self.k_scale = torch.zeros(L, H, D, dtype=torch.float32, device=dev)
            self.v_scale = torch.zeros(L, H, cap_blocks, dtype=torch.float32, device=dev)
        elif kv_format == "int8_token":
            self.k_tscale = torch.zeros(L, H, cap_blocks * B, dtype=torch.float16, device=dev)
            self.v_tscale = torch.zeros_like(self.k_tscale)
        self.desc = _lib.NkvStore(
            hist_k_addr, hist_v_addr, _ptr(self.reps).value,
            _ptr(self.sink_k).value, _ptr(self.sink_v).value,
            _ptr(self.recent_k).value, _ptr(self.recent_v).value,
            _ptr(self.k_scale).value, _ptr(self.v_scale).value,
            _ptr(self.k_tscale).value, _ptr(self.v_tscale).value,
            L, num_heads, num_kv_heads, D, B, r, cap_blocks, S, R, KV_FORMATS[kv_format])
        self._desc_ref = ctypes.byref(self.desc)

    # ------------------------------------------------------------------
    @staticmethod
    def _bf16(t, name):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
        if not t.is_cuda:
            raise ValueError(f"{name} must be a device tensor")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        return t

    def store_chunk(self, layer0: int, k, v, start_block: int, compute_k_scale: bool,
                    write_sink: bool) -> None:
        """History (+ int8 scales) and sink for a chunk k, v: [nl, T, Hkv, D]."""
        self._bf16(k, "k")
        self._bf16(v, "v")
        nl, T = k.shape[0], k.shape[1]
        _lib.check(self.lib.nkv_store_chunk(
            self._desc_ref, layer0, nl, _ptr(k), _ptr(v), k.stride(0), T, start_block,
            int(compute_k_scale), int(write_sink), _stream()), "store_chunk")

    def build_reps(self, layer0: int, k, start_block: int) -> None:
        self._bf16(k, "k")
        _lib.check(self.lib.nkv_build_reps(
            self._desc_ref, layer0, k.shape[0], _ptr(k), k.stride(0), k.shape[1], start_block,
            _stream()), "build_reps")

    def recent_update(self, layer0: int, nl: int, k, v, src_lo: int, n_src: int,
                      ring_start: int, old_len: int, carry: int) -> None:
        if n_src:
            self._bf16(k, "k")
            self._bf16(v, "v")
        _lib.check(self.lib.nkv_recent_update(
            self._desc_ref, layer0, nl, _ptr(k if n_src else None), _ptr(v if n_src else None),
            k.stride(0) if n_src else 0, src_lo, n_src, ring_start, old_len, carry, _stream()),
            "recent_update")

    def select(self, layer0: int, q, nblocks: int, prot_dev, n_prot: int, k: int, order: int,
               per_query: bool, score_keys, out_scores, out_ids, out_vals) -> None:
        """score_keys: zeroed uint32 workspace of nl * nq' * nblocks words (left
        zeroed), nq' = nq if per_query else 1; out_scores may be None."""
        self._bf16(q, "q")
        nl, nq = q.shape[0], q.shape[1]
        need = nl * (nq if per_query else 1) * nblocks
        if score_keys.numel() < need or score_keys.dtype not in (torch.int32, torch.uint32):
            raise ValueError(f"select: score_keys needs {need} 32-bit words, got {score_keys.numel()}")
        _lib.check(self.lib.nkv_select(
            self._desc_ref, layer0, nl, _ptr(q), q.stride(0), nq, int(per_query), nblocks,
            _ptr(prot_dev), n_prot, k, order, _ptr(score_keys), _ptr(out_scores), _ptr(out_ids),
            _ptr(out_vals), _stream()), "select")

    def attend(self, layer0: int, q, k_new, v_new, n_chunk: int,
               write_slot: int, ids, ids_layer_stride: int, n_hist: int, allowed,
               sink_len: int, ring_base: int, rec_lo: int, rec_len: int, scale: float,
               splits: int, partial_ws, out, allowed_layer_stride: int = 0) -> None:
        self._bf16(q, "q")
        self._bf16(out, "out")
        nl, tq = q.shape[0], q.shape[1]
        kv_stride = k_new.stride(0) if k_new is not None else 0
        _lib.check(self.lib.nkv_attend(
            self._desc_ref, layer0, nl, _ptr(q), q.stride(0), tq, _ptr(k_new), _ptr(v_new),
            kv_stride, n_chunk, write_slot, _ptr(ids), ids_layer_stride, n_hist,
            _ptr(allowed), allowed_layer_stride, sink_len, ring_base, rec_lo, rec_len, float(scale),
            splits, _ptr(partial_ws), _ptr(out), _stream()), "attend")

    def prefill_attend(self, layer0: int, q, k_new, v_new, ids, ids_layer_stride: int,
                       n_hist: int, allowed, sink_len: int, ring_base: int, rec_lo: int,
                       rec_len: int, scale: float, out, allowed_layer_stride: int = 0,
                       splits: int = 1, partial_ws=None) -> None:
        """Many-query causal attention on the matrix cores (chunk = the queries' own tokens)."""
        self._bf16(q, "q")
        self._bf16(out, "out")
        nl, tq = q.shape[0], q.shape[1]
        _lib.check(self.lib.nkv_prefill_attend(
            self._desc_ref, layer0, nl, _ptr(q), q.stride(0), tq, _ptr(k_new), _ptr(v_new),
            k_new.stride(0), _ptr(ids), ids_layer_stride, n_hist, _ptr(allowed),
            allowed_layer_stride, sink_len, ring_base, rec_lo, rec_len, float(scale), splits,
            _ptr(partial_ws), _ptr(out), _stream()), "prefill_attend")

    def prefill_attend_tiled(self, layer0: int, q, k_new, v_new, ids, ids_layer_stride: int,
                             ids_tile_stride: int, sel_tile: int, n_hist: int, sink_len: int, ring_base: int,
                             rec_lo: int, rec_len: int, scale: float, out, splits: int = 1, partial=None) -> None:
        """nkv_prefill_attend_tiled: one history selection per tile of sel_tile queries."""
        self._bf16(q, "q")
        self._bf16(out, "out")
        if ids.dtype != torch.int32 or not ids.is_contiguous():
            raise ValueError("prefill_attend_tiled: ids must be contiguous int32")
        nl, tq = q.shape[0], q.shape[1]
        _lib.check(self.lib.nkv_prefill_attend_tiled(
            self._desc_ref, layer0, nl, _ptr(q), q.stride(0), tq, _ptr(k_new), _ptr(v_new), k_new.stride(0),
            _ptr(ids), ids_layer_stride, ids_tile_stride, sel_tile, n_hist, sink_len, ring_base, rec_lo, rec_len,
            float(scale), splits, _ptr(partial), _ptr(out), _stream()), "prefill_attend_tiled")

    def prefill_workspace_floats(self, nl: int, tq: int, splits: int) -> int:
        return int(self.lib.nkv_prefill_workspace_floats(nl, self.num_kv_heads, self.num_heads,
                                                         tq, splits))

    def select_union(self, ids, k_eff: int, umax: int, out_union, out_count, out_allowed) -> None:
        """nkv_select_union: ids [L, tq, k] int32 per-query selections -> union [L, umax]
        (ascending, -1 padded), counts [L], allowed [L, tq, umax] uint8."""
        nl, tq, k = ids.shape
        if not ids.is_contiguous() or ids.dtype != torch.int32:
            raise ValueError("select_union: ids must be contiguous int32 [L, tq, k]")
        if (out_union.numel() < nl * umax or out_count.numel() < nl
                or out_allowed.numel() < nl * tq * umax):
            raise ValueError("select_union: output buffers too small")
        _lib.check(self.lib.nkv_select_union(_ptr(ids), nl, tq, k, k_eff, umax, _ptr(out_union),
                                             _ptr(out_count), _ptr(out_allowed), _stream()),
                   "select_union")

    def select_per_query(self, layer0: int, q, nblocks: int, prot_dev, n_prot: int, k: int, score_keys,
                         out_scores, out_ids, out_vals, umax: int, out_union, out_count, out_allowed) -> None:
        """nkv_select_per_query: select(per_query=True) and select_union in two launches
        (q [L, nq, Hq, D] with nq <= 16, k <= 64, nblocks <= 2048)."""
        self._bf16(q, "q")
        nl, nq = q.shape[0], q.shape[1]
        need = nl * nq * nblocks
        if score_keys.numel() < need or score_keys.dtype not in (torch.int32, torch.uint32):
            raise ValueError(f"select_per_query: score_keys needs {need} 32-bit words, got {score_keys.numel()}")
        if (out_ids.numel() < nl * nq * k or out_union.numel() < nl * umax or out_count.numel() < nl
                or out_allowed.numel() < nl * nq * umax):
            raise ValueError("select_per_query: output buffers too small")
        _lib.check(self.lib.nkv_select_per_query(
            self._desc_ref, layer0, nl, _ptr(q), q.stride(0), nq, nblocks, _ptr(prot_dev), n_prot, k,
            _ptr(score_keys), _ptr(out_scores), _ptr(out_ids), _ptr(out_vals), umax, _ptr(out_union),
            _ptr(out_count), _ptr(out_allowed), _stream()), "select_per_query")

    def attend_workspace_floats(self, nl: int, tq: int, splits: int) -> int:
        return int(self.lib.nkv_attend_workspace_floats(nl, self.num_kv_heads, self.num_heads,
                                                        tq, splits))

    def decode_step(self, layer0: int, q, k_new, v_new, nblocks: int, prot_dev, n_prot: int,
                    k: int, n_hist: int, sink_len: int, write_slot: int, ring_base: int,
                    rec_lo: int, rec_len: int, scale: float, splits: int, score_keys, out_ids,
                    partial_ws, out, streams) -> None:
        """nkv_decode_step: selection + attention for q.shape[0] layers, the layer
        ranges on `streams` (raw stream handles, the caller's first)."""
        self._bf16(q, "q")
        self._bf16(out, "out")
        nl = q.shape[0]
        if not (q.is_contiguous() and k_new.is_contiguous() and v_new.is_contiguous()
                and out.is_contiguous() and out_ids.is_contiguous()):
            raise ValueError("decode_step: q, k_new, v_new, out and out_ids must be contiguous")
        if q.shape[1] != 1 or k_new.shape[:2] != (nl, 1) or out.shape != q.shape:
            raise ValueError("decode_step: expects q/out [L, 1, Hq, D] and k/v [L, 1, Hkv, D]")
        if out_ids.numel() < nl * k or score_keys.numel() < nl * nblocks:
            raise ValueError("decode_step: out_ids or score_keys too small")
        arr = (ctypes.c_void_p * len(streams))(*streams)
        _lib.check(self.lib.nkv_decode_step(
            self._desc_ref, layer0, nl, _ptr(q), _ptr(k_new), _ptr(v_new), nblocks, _ptr(prot_dev),
            n_prot, k, n_hist, sink_len, write_slot, ring_base, rec_lo, rec_len, float(scale), splits,
            _ptr(score_keys), _ptr(out_ids), _ptr(partial_ws), _ptr(out), len(streams), arr),
            "decode_step")

    def decode_step_ring(self, layer0: int, q, k_new, v_new, nblocks: int, prot_dev, n_prot: int, k: int,
                         n_hist: int, sink_len: int, ring_start, scale: float, splits: int, score_keys, out_ids,
                         partial_ws, out) -> None:
        """nkv_decode_step_ring: the steady-state decode step of q.shape[0] layers with
        their ring starts in `ring_start` (int32 [L] on the device, advanced by the call)."""
        self._bf16(q, "q")
        self._bf16(out, "out")
        nl = q.shape[0]
        if not (q.is_contiguous() and k_new.is_contiguous() and v_new.is_contiguous()
                and out.is_contiguous() and out_ids.is_contiguous()):
            raise ValueError("decode_step_ring: q, k_new, v_new, out and out_ids must be contiguous")
        if q.shape[1] != 1 or k_new.shape[:2] != (nl, 1) or out.shape != q.shape:
            raise ValueError("decode_step_ring: expects q/out [L, 1, Hq, D] and k/v [L, 1, Hkv, D]")
        if out_ids.numel() < nl * k or score_keys.numel() < nl * nblocks:
            raise ValueError("decode_step_ring: out_ids or score_keys too small")
        if ring_start.dtype != torch.int32 or ring_start.numel() < nl or ring_start.device != q.device:
            raise ValueError("decode_step_ring: ring_start must be int32 with one entry per layer, on q's device")
        _lib.check(self.lib.nkv_decode_step_ring(
            self._desc_ref, layer0, nl, _ptr(q), _ptr(k_new), _ptr(v_new), nblocks, _ptr(prot_dev), n_prot, k,
            n_hist, sink_len, _ptr(ring_start), float(scale), splits, _ptr(score_keys), _ptr(out_ids),
            _ptr(partial_ws), _ptr(out), _stream()), "decode_step_ring")

    def decode_step_workspace_floats(self, nl: int, splits: int, nstreams: int) -> int:
        return int(self.lib.nkv_decode_step_workspace_floats(nl, self.num_kv_heads, self.num_heads,
                                                             splits, nstreams))


def query_summaries(q, nsegments: int):
    """prefill_query_summaries on device: q [nl, T, Hq, D] -> [nl, nseg, Hq, D] bf16."""
    lib = _lib.load()
    SparseKVStore._bf16(q, "q")
    nl, T, hq, d = q.shape
    nseg = min(nsegments, T)
    out = torch.empty(nl, nseg, hq, d, dtype=torch.bfloat16, device=q.device)
    _lib.check(lib.nkv_query_summaries(_ptr(q), q.stride(0), nl, T, hq, d, nsegments, _ptr(out),
                                       out.stride(0), _stream()), "query_summaries")
    return out


def tile_summaries(q, tile: int):
    """Per-tile query means of a chunk: q [nl, T, Hq, D] -> [nl, ceil(T / tile), Hq, D]
    bf16; tile i is queries [i * tile, min(T, (i + 1) * tile)) (the last tile
    may be shorter), each mean rounded as prefill_query_summaries rounds."""
    lib = _lib.load()
    SparseKVStore._bf16(q, "q")
    nl, T, hq, d = q.shape
    nfull, rem = divmod(T, tile)
    out = torch.empty(nl, nfull + (1 if rem else 0), hq, d, dtype=torch.bfloat16, device=q.device)
    if nfull:
        _lib.check(lib.nkv_query_summaries(_ptr(q), q.stride(0), nl, nfull * tile, hq, d, nfull, _ptr(out),
                                           out.stride(0), _stream()), "query_summaries")
    if rem:
        tail = ctypes.c_void_p(q.data_ptr() + nfull * tile * q.stride(1) * q.element_size())
        dst = ctypes.c_void_p(out.data_ptr() + nfull * out.stride(1) * out.element_size())
        _lib.check(lib.nkv_query_summaries(tail, q.stride(0), nl, rem, hq, d, 1, dst, out.stride(0), _stream()),
                   "query_summaries")
    return out


def packed_attention(q, k, v, causal_from: int, scale: float, mask=None, splits: int | None = None):
    """Exact attention over caller-packed keys on the device (nkv_attend_packed).

    q [Tq, Hq, 128], k / v [S, Hkv, 128] bf16 (token-major); query t sees key
    j iff j - causal_from <= t and mask[t, j] is False (mask: bool / uint8
    [Tq, S], True = hidden, or None) -> [Tq, Hq, 128] bf16.
    """
    lib = _lib.load()
    q = SparseKVStore._bf16(q.contiguous(), "q")
    k = SparseKVStore._bf16(k.contiguous(), "k")
    v = SparseKVStore._bf16(v.contiguous(), "v")
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or q.shape[-1] != HEAD_DIM or k.shape[-1] != HEAD_DIM:
        raise ValueError(f"packed attention needs q [Tq, Hq, {HEAD_DIM}] and k = v [S, Hkv, {HEAD_DIM}] "
                         f"(got q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)})")
    if not (q.device == k.device == v.device) or q.device.type != "cuda":
        raise ValueError("packed attention: q, k and v must be on one GPU")
    tq, hq, _ = q.shape
    s_len, hkv, _ = k.shape
    if hq % hkv:
        raise ValueError(f"num_heads {hq} is not a multiple of num_kv_heads {hkv}")
    g = hq // hkv
    m8 = None
    if mask is not None:
        if tuple(mask.shape) != (tq, s_len):
            raise ValueError(f"attn_mask must be [{tq}, {s_len}] (got {tuple(mask.shape)})")
        m8 = mask.to(device=q.device, dtype=torch.uint8).contiguous()
    nseg = -(-s_len // BLOCK_SIZE)
    if splits is None:
        if tq * g > 16:   # matrix-core kernel: ~1536 workgroups, >= 4 segments per split
            tiles = -(-tq // (128 // g)) * hkv
            splits = max(1, min(round(1536 / tiles), nseg // 4, 64))
        else:             # few-query kernel: ~1440 workgroups, >= 4 segments per split
            groups = -(-tq // max(1, min(tq, 16 // g))) * hkv
            splits = max(1, min(round(1440 / groups), -(-nseg // 4), 64))
    ws = int(lib.nkv_attend_packed_workspace_floats(hq, hkv, tq, splits))
    part = torch.empty(max(ws, 1), dtype=torch.float32, device=q.device) if ws else None
    out = torch.empty_like(q)
    _lib.check(lib.nkv_attend_packed(hq, hkv, _ptr(q), tq, _ptr(k), _ptr(v), s_len, int(causal_from), _ptr(m8),
                                     float(scale), splits, _ptr(part), _ptr(out), _stream()), "attend_packed")
    return out
