"""CPU oracle for the NanoKV sparse-attention layer-step (TEST INFRASTRUCTURE).

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``nanokv_amd``) runs hand-written HIP kernels and
raises when the HIP library is missing; it never calls into this file.

It restates, in numpy, the semantics of the reference's M12 sparse runtime
(``nanovllm/sparse/m12_runtime.py``), its Triton scorer and dequant kernels
(``nanovllm/sparse/fused_select.py``, ``nanovllm/sparse/fused_dequant.py``),
the int8 scheme (``nanovllm/sparse/quant_kv.py``) and the GQA / attention
oracles of ``nanovllm/sparse/block_sparse.py``.  Each function names the
reference lines it follows.

Numeric definitions that the reference leaves open (it uses torch's fp32
einsum, whose summation order is unspecified, and ``torch.topk``, whose tie
order is unspecified) are fixed here and shared with the HIP kernels:

* block score: each 128-term dot product ``q . rep`` is accumulated in fp32 in
  ascending ``d`` order, ``acc = fma(q[d], rep[d], acc)`` from ``acc = +0``.
  A bf16 x bf16 product is exact in fp32, so this equals
  ``acc = fl32(acc + q[d]*rep[d])`` and is reproduced bit-for-bit below;
* Top-K order: score descending, block id ascending on exact ties, NaN above
  +inf (torch's NaN-is-largest convention), ``-0.0`` treated as ``+0.0``;
* query-summary mean: bf16 round-to-nearest-even of the fp64 mean.

Pinning (which checks hold each function) is listed per function and
enforced by ``tests/test_oracle_pins.py``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

F32 = np.float32
QMAX = 127  # nanovllm/sparse/quant_kv.py:24


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------

def bf16_round(x) -> np.ndarray:
    """Round fp32 values to bf16 (round-to-nearest-even); float32 result.

    Same rounding as ``tensor.to(torch.bfloat16)``.  Pinned by hand-made
    halfway cases in the oracle tests.
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=F32))
    u = a.view(np.uint32).astype(np.uint64)
    bias = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    r = (((u + bias) >> np.uint64(16)) << np.uint64(16)).astype(np.uint32)
    out = r.view(F32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of bf16-representable float32 values."""
    a = np.ascontiguousarray(bf16_round(x))
    return (a.view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << np.uint32(16)).view(F32)


def f64_to_bf16(x) -> np.ndarray:
    """Round fp64 values directly to bf16 (RNE, one rounding); float32 result."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
    u = a.view(np.uint64)
    # bf16 keeps the top 16 bits of the fp32 pattern = sign, 8-bit exponent,
    # 7 mantissa bits.  Go through the exact fp64 value: scale the mantissa so
    # the 8 significant bits become an integer, round-half-even, rebuild.
    out = np.empty(a.shape, dtype=F32)
    flat_in = a.reshape(-1)
    flat_out = out.reshape(-1)
    for i, v in enumerate(flat_in):
        if not math.isfinite(v) or v == 0.0:
            flat_out[i] = F32(v)
            continue
        m, e = math.frexp(v)            # v = m * 2**e, 0.5 <= |m| < 1
        if e - 1 < -126:                # bf16 subnormal range: fixed quantum 2**-133
            q = round(v * 2.0 ** 133)   # Python round = half-to-even
            flat_out[i] = F32(q * 2.0 ** -133)
            continue
        q = round(m * 256.0)            # 8 significant bits, half-to-even
        flat_out[i] = F32(math.ldexp(q, e - 8))
    del u
    return out


# ---------------------------------------------------------------------------
# GQA map and bookkeeping helpers
# ---------------------------------------------------------------------------

def kv_head_for_query(num_query_heads: int, num_kv_heads: int) -> np.ndarray:
    """GQA map h -> h // (Hq/Hkv).  nanovllm/sparse/block_sparse.py:33-41."""
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be divisible by num_kv_heads")
    return np.arange(num_query_heads) // (num_query_heads // num_kv_heads)


def prefill_recent_slice(valid_len: int, sink_tokens: int, recent_tokens: int):
    """(buffer_start, buffer_offset, length).  m12_runtime.py:32-50.

    Pinned by the reference's known answers (tests/test_m14_prefill_layout.py:34-44).
    """
    assert valid_len >= 0 and sink_tokens >= 0 and recent_tokens >= 0
    sink_len = min(sink_tokens, valid_len)
    buffer_len = min(recent_tokens, valid_len)
    buffer_start = valid_len - buffer_len
    include_start = max(sink_len, buffer_start)
    return buffer_start, include_start - buffer_start, valid_len - include_start


def protected_blocks_after_store(nblocks: int, recent_tokens: int, block_size: int) -> set:
    """{0} U [max(1, nb - R/B), nb).  m12_runtime.py:509-513."""
    n_recent_blocks = recent_tokens // block_size
    return {0} | set(range(max(1, nblocks - n_recent_blocks), nblocks))


def tensor_split_bounds(total: int, n: int):
    """Bounds of torch.tensor_split(x, n) along dim 0 (first total % n parts are longer)."""
    base, extra = divmod(total, n)
    bounds, start = [], 0
    for i in range(n):
        size = base + (1 if i < extra else 0)
        bounds.append((start, start + size))
        start += size
    return bounds


def query_summaries(q, nsegments: int) -> np.ndarray:
    """prefill_query_summaries (m12_runtime.py:53-67): segment means of q.

    q: [T, Hq, D] bf16-valued.  Each mean is the bf16 RNE rounding of the fp64
    mean (the fp64 sum of bf16 values is exact here), shape [n, Hq, D].
    """
    q = np.asarray(q, dtype=F32)
    assert q.ndim == 3 and nsegments > 0
    nseg = min(nsegments, q.shape[0])
    outs = []
    for lo, hi in tensor_split_bounds(q.shape[0], nseg):
        s = q[lo:hi].astype(np.float64).sum(axis=0)
        outs.append(f64_to_bf16(s / float(hi - lo)))
    return np.stack(outs)


# ---------------------------------------------------------------------------
# Scoring (kernel 1) -- fused_select.py:23-54, m12_runtime.py:999-1003
# ---------------------------------------------------------------------------

def _rep_dots(q, reps, nblocks, num_kv_heads):
    """fp32 sequential-FMA dots [Nq, Hkv, G, nb, r] (definition in module doc)."""
    q = np.asarray(q, dtype=F32)
    if q.ndim == 2:
        q = q[None]
    nq, hq, d = q.shape
    g = hq // num_kv_heads
    qg = q.reshape(nq, num_kv_heads, g, d)
    rp = np.asarray(reps, dtype=F32)[:, :nblocks]          # [Hkv, nb, r, D]
    acc = np.zeros((nq, num_kv_heads, g, nblocks, rp.shape[2]), dtype=F32)
    for i in range(d):
        prod = qg[:, :, :, i][:, :, :, None, None] * rp[None, :, None, :, :, i]
        acc = (acc + prod).astype(F32)
    return acc


def block_scores(q, reps, nblocks: int, num_kv_heads: int) -> np.ndarray:
    """score[b] = max over (n, h, g, j) of q[n, h*G+g] . reps[h, b, j].

    Reference: fused_select.py:23-54 (Triton) and the eager chain
    m12_runtime.py:999-1003 (einsum "nhgd,hbrd->nhgbr" -> amax r, G, n, Hkv).
    Pinned: exact rational sums (fractions) within the fp32 bound, and a
    pure-Python sequential loop, in tests/test_oracle_pins.py.
    """
    if nblocks == 0:
        return np.zeros(0, dtype=F32)
    return _rep_dots(q, reps, nblocks, num_kv_heads).max(axis=(0, 1, 2, 4))


def block_scores_per_query(q, reps, nblocks: int, num_kv_heads: int) -> np.ndarray:
    """gs[t, b] = max over (h, g, j).  m12_runtime.py:1068-1072."""
    return _rep_dots(q, reps, nblocks, num_kv_heads).max(axis=(1, 2, 4))


# ---------------------------------------------------------------------------
# Top-K (kernel 2) -- m12_runtime.py:982-988, :1004-1014, :1033
# ---------------------------------------------------------------------------

def orderable_key(scores) -> np.ndarray:
    """Monotone uint32 key of fp32 scores (-0 folded onto +0, NaN largest)."""
    s = np.asarray(scores, dtype=F32) + F32(0.0)          # -0.0 + 0.0 = +0.0
    u = np.ascontiguousarray(s).view(np.uint32)
    nan = np.isnan(s)
    u = np.where(nan, np.uint32(0x7FC00000), u)           # canonical quiet NaN
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def effective_k(nblocks: int, protected, requested: int) -> int:
    """k = min(requested, max(1, nb - |protected in range|)).  m12_runtime.py:982-988."""
    n_prot = len([p for p in protected if 0 <= p < nblocks])
    return min(int(requested), max(1, nblocks - n_prot))


def topk_blocks(scores, protected, requested: int):
    """Protected -> -inf, then Top-k sorted (score desc, id asc).

    Returns (ids int64 [k], values f32 [k]).  Reference: m12_runtime.py:1004-1014
    (protected mask), :1033 (``global_scores.topk(k)``).  The id-ascending tie
    rule replaces torch.topk's unspecified tie order.
    Pinned: brute-force sorted() on small inputs plus the reference known
    answers (test_block_sparse.py:156-161, test_m16_dynamic_topk.py:26-43,
    test_m19_selector_graph.py:47-87).
    """
    s = np.array(scores, dtype=F32, copy=True)
    nb = s.shape[0]
    if nb == 0:
        raise ValueError("selection needs at least one history block")
    prot = [p for p in protected if 0 <= p < nb]
    if prot:
        s[np.asarray(sorted(prot))] = F32(-np.inf)
    k = effective_k(nb, protected, requested)
    key = orderable_key(s).astype(np.int64)
    order = np.lexsort((np.arange(nb), -key))
    ids = order[:k].astype(np.int64)
    return ids, s[ids]


def select_blocks(q, reps, nblocks, num_kv_heads, protected, requested):
    """_gpu_select fixed-budget path (m12_runtime.py:959-1055) -> (ids, values)."""
    return topk_blocks(block_scores(q, reps, nblocks, num_kv_heads), protected, requested)


def select_per_query(q, reps, nblocks, num_kv_heads, protected, k):
    """_gpu_select_per_query (m12_runtime.py:1057-1087).

    Returns (union ids sorted ascending [U], allowed bool [Tq, U], per-query ids [Tq, kk]).
    """
    gs = block_scores_per_query(q, reps, nblocks, num_kv_heads)
    kk = effective_k(nblocks, protected, k)
    tops = np.stack([topk_blocks(gs[t], protected, kk)[0] for t in range(gs.shape[0])])
    union = np.unique(tops.reshape(-1))
    allowed = np.zeros((gs.shape[0], union.shape[0]), dtype=bool)
    for t in range(gs.shape[0]):
        allowed[t, np.searchsorted(union, tops[t])] = True
    return union.astype(np.int64), allowed, tops


def dynamic_top_k_from_scores(top_scores, max_k: int, target_mass: float) -> int:
    """Budget in {half, 3/4, all} by softmax mass.  m12_runtime.py:70-95."""
    ts = np.asarray(top_scores, dtype=F32)
    assert ts.ndim == 1 and 0.0 < target_mass <= 1.0 and max_k > 0
    count = ts.shape[0]
    if count < max_k or count <= 1 or not np.isfinite(ts).all():
        return count
    scale = ts.astype(np.float64).std()
    if scale <= 1e-6:
        return count
    w = np.exp((ts - ts[0]) / scale)
    w = w / w.sum()
    cum = np.cumsum(w)
    for choice in sorted({max(1, (max_k + 1) // 2), max(1, (3 * max_k + 3) // 4), max_k}):
        if cum[choice - 1] >= target_mass:
            return choice
    return max_k


def relative_threshold_select(scores, protected, requested: int, a: float, scale: float,
                              max_blocks: int, union: bool):
    """Relative-threshold decode selection (m12_runtime.py:1015-1031).

    Protected -> -inf; threshold = max score + ln(a) / scale; among the first
    cap = min(max_blocks, max(1, avail)) blocks in (score desc, id asc) order,
    keep those with score >= threshold (with ``union``: also the first k of
    them); if none is kept, the first k.  Returns (ids int64, values f32) in
    score order.  k = effective_k(...).  Pinned by hand-computed known answers
    in tests/test_oracle_pins.py.
    """
    s = np.array(scores, dtype=F32, copy=True)
    nb = s.shape[0]
    prot = [p for p in protected if 0 <= p < nb]
    if prot:
        s[np.asarray(sorted(prot))] = F32(-np.inf)
    avail = nb - len(prot)
    k = effective_k(nb, protected, requested)
    cap = min(int(max_blocks), max(1, avail))
    key = orderable_key(s).astype(np.int64)
    order = np.lexsort((np.arange(nb), -key))
    threshold = float(s.max()) + math.log(a) / scale
    cand = order[:cap]
    keep = s[cand] >= threshold
    if union:
        keep = keep | (np.arange(cand.shape[0]) < k)
    if not keep.any():
        ids = order[:k]
    else:
        ids = cand[keep]
    return ids.astype(np.int64), s[ids]


# ---------------------------------------------------------------------------
# Representatives -- m12_runtime.py:354-395
# ---------------------------------------------------------------------------

def build_reps(k_blocks, r: int):
    """r real-key representatives per (block, KV head).

    k_blocks: [N, B, Hkv, D] bf16-valued.  Returns (sel_idx int64 [N, Hkv, r],
    reps [Hkv, N, r, D] float32, margins [N, Hkv, r] float64).  Follows
    m12_runtime.py:354-395 in fp64: normalise each key (norm clamped to
    1e-12), seed = first argmax of cos to the normalised mean direction, then
    r-1 farthest-point steps: first argmin over tokens of the max cos to the
    chosen set, chosen tokens forced to 2.0.  ``margins`` is the gap between
    the winning and the runner-up value of each argmax/argmin, so a test can
    tell a genuine tie-break disagreement from a real bug.
    Pinned: a pure-Python loop restatement on tiny inputs and the invariants
    in tests/test_oracle_pins.py.
    """
    K = np.asarray(k_blocks, dtype=np.float64)
    N, B, H, D = K.shape
    norm = np.sqrt((K * K).sum(axis=-1, keepdims=True))
    Kd = K / np.maximum(norm, 1e-12)
    mean = Kd.mean(axis=1)                                   # [N, H, D]
    mnorm = np.sqrt((mean * mean).sum(axis=-1, keepdims=True))
    mean_dir = mean / np.maximum(mnorm, 1e-12)
    cos0 = np.einsum("nbhd,nhd->nbh", Kd, mean_dir)          # [N, B, H]
    sel = np.zeros((N, H, r), dtype=np.int64)
    margins = np.zeros((N, H, r), dtype=np.float64)
    sel[:, :, 0] = cos0.argmax(axis=1)
    srt = np.sort(cos0, axis=1)
    margins[:, :, 0] = srt[:, -1, :] - srt[:, -2, :] if B > 1 else np.inf
    for step in range(1, r):
        maxcos = np.full((N, B, H), -np.inf)
        for s in range(step):
            idx = sel[:, :, s]                                   # [N, H]
            dirs = np.take_along_axis(Kd, idx[:, None, :, None], axis=1)[:, 0]  # [N, H, D]
            maxcos = np.maximum(maxcos, np.einsum("nbhd,nhd->nbh", Kd, dirs))
        for s in range(step):
            idx = sel[:, :, s]
            n_i, h_i = np.meshgrid(np.arange(N), np.arange(H), indexing="ij")
            maxcos[n_i, idx, h_i] = np.maximum(maxcos[n_i, idx, h_i], 2.0)
        sel[:, :, step] = maxcos.argmin(axis=1)
        srt = np.sort(maxcos, axis=1)
        margins[:, :, step] = srt[:, 1, :] - srt[:, 0, :] if B > 1 else np.inf
    Kf = np.asarray(k_blocks, dtype=F32)
    reps = np.take_along_axis(Kf.transpose(0, 2, 1, 3), sel[..., None], axis=2)  # [N, H, r, D]
    return sel, reps.transpose(1, 0, 2, 3).copy(), margins


# ---------------------------------------------------------------------------
# int8 scheme -- quant_kv.py:24-63, m12_runtime.py:460-477, fused_dequant.py:24-44
# ---------------------------------------------------------------------------

def k_scale_from_chunk(k_blocks) -> np.ndarray:
    """[Hkv, D] fp32 = max(amax|k| over (blocks, tokens), 1e-8) / 127.  m12_runtime.py:463-467."""
    a = np.abs(np.asarray(k_blocks, dtype=F32)).max(axis=(0, 1))
    return (np.maximum(a, F32(1e-8)) / F32(QMAX)).astype(F32)


def quantize(x, scale) -> np.ndarray:
    """round-half-even(x / scale) clamped to +-127, int8.  quant_kv.py:27-49."""
    q = np.rint((np.asarray(x, dtype=F32) / np.asarray(scale, dtype=F32)).astype(F32))
    return np.clip(q, -QMAX, QMAX).astype(np.int8)


def v_scale_per_block(v_blocks) -> np.ndarray:
    """[N, Hkv] fp32 = max(amax|v| over (tokens, D), 1e-8) / 127.  m12_runtime.py:469-474."""
    a = np.abs(np.asarray(v_blocks, dtype=F32)).max(axis=(1, 3))
    return (np.maximum(a, F32(1e-8)) / F32(QMAX)).astype(F32)


def dequant_to_bf16(q, scale) -> np.ndarray:
    """bf16(int8 * scale) as the reference packs it (m12_runtime.py:1262-1267, fused_dequant.py:34-44)."""
    return bf16_round(np.asarray(q, dtype=F32) * np.asarray(scale, dtype=F32))


def token_scale_fp16(x) -> np.ndarray:
    """Per-token-per-KV-head fp16 scale for the [T, Hkv, D] layout.

    scale = fp16(max(amax_d |x| / 127, 2**-24)): the fp32 quotient is rounded
    once to fp16; the floor 2**-24 is the smallest fp16 subnormal, so an
    all-zero row still gets a non-zero scale.  This layout is the second
    scale scheme of the int8 workload (the reference has only the
    per-channel / per-block one).  Pinned by closed form in the oracle tests.
    """
    a = np.abs(np.asarray(x, dtype=F32)).max(axis=-1)
    s32 = np.maximum((a / F32(QMAX)).astype(F32), F32(2.0 ** -24))
    return s32.astype(np.float16)


# ---------------------------------------------------------------------------
# Attention -- m12_runtime.py:845-896, block_sparse.py:153-208
# ---------------------------------------------------------------------------

def attention_fp64(q, k, v, scale: float, mask=None) -> np.ndarray:
    """softmax(q K^T * scale) V per GQA group, fp64.  mask [Tq, S] True = disallowed.

    Same math as m12_runtime.py:867-873 (fast path) and :875-896 (masked),
    evaluated in fp64 so the only difference to the reference's fp32 einsum
    is the reference's own rounding.  Pinned by block_sparse's textbook
    identities (test_block_sparse.py:36-49, :236-242) in the oracle tests.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    tq, hq, d = q.shape
    s_len, hkv, _ = k.shape
    g = hq // hkv
    qg = q.reshape(tq, hkv, g, d)
    logits = np.einsum("thgd,shd->thgs", qg, k) * scale
    if mask is not None:
        logits = np.where(np.asarray(mask)[:, None, None, :], -np.inf, logits)
    mx = logits.max(axis=-1, keepdims=True)
    p = np.exp(logits - mx)
    p = p / p.sum(axis=-1, keepdims=True)
    out = np.einsum("thgs,shd->thgd", p, v)
    return out.reshape(tq, hq, d)


def attention_bf16_probs(q, k, v, scale: float, mask=None) -> np.ndarray:
    """attention_fp64 with the probabilities rounded to bf16 before P.V.

    The numerics class of flash attention with bf16 operands, which the
    reference's prefill runs (flash_attn_func, m12_runtime.py:834-839): P is
    fed to the P.V product in bf16, the normaliser sums the unrounded P.
    Used only to size the tolerance of the matrix-core prefill kernel.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    tq, hq, d = q.shape
    s_len, hkv, _ = k.shape
    g = hq // hkv
    logits = np.einsum("thgd,shd->thgs", q.reshape(tq, hkv, g, d), k) * scale
    if mask is not None:
        logits = np.where(np.asarray(mask)[:, None, None, :], -np.inf, logits)
    p = np.exp(logits - logits.max(axis=-1, keepdims=True))
    pb = bf16_round(p.astype(F32)).astype(np.float64)
    out = np.einsum("thgs,shd->thgd", pb, v) / p.sum(axis=-1, keepdims=True)
    return out.reshape(tq, hq, d)


def lossless_history_mask(allowed, block_size: int, s_len: int) -> np.ndarray:
    """Per-query mask of lossless verify (m12_runtime.py:746-748): True =
    disallowed.  allowed [Tq, U] says query t may read union block j; block j
    occupies packed keys [j*B, (j+1)*B), so its flag repeats B times along the
    key axis; keys past the U*B history tokens (sink, recent, chunk) are not
    masked here."""
    allowed = np.asarray(allowed, dtype=bool)
    m = np.zeros((allowed.shape[0], s_len), dtype=bool)
    m[:, :allowed.shape[1] * block_size] = ~np.repeat(allowed, block_size, axis=1)
    return m


def causal_mask(tq: int, s_len: int, causal_from: int, attn_mask=None) -> np.ndarray:
    """mask[t, s] = (s >= t + causal_from + 1) & (s >= causal_from), OR attn_mask.

    m12_runtime.py:877-883.
    """
    cols = np.arange(s_len)[None, :]
    rows = (np.arange(tq) + causal_from + 1)[:, None]
    m = (cols >= rows) & (cols >= causal_from)
    if attn_mask is not None:
        m = m | np.asarray(attn_mask, dtype=bool)
    return m


# ---------------------------------------------------------------------------
# Whole-runtime state machine -- M12LayerRuntime semantics
# ---------------------------------------------------------------------------

@dataclass
class OracleConfig:
    """Subset of M12Config (m12_runtime.py:98-166) that the layer-step reads."""
    block_size: int = 64
    r: int = 4
    recent_tokens: int = 512
    sink_tokens: int = 64
    top_k_blocks: int = 32
    prefill_top_k_blocks: int | None = None
    decode_top_k_blocks: int | None = None
    quant_history: bool = False
    prefill_query_segments: int = 1
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    scale: float = 128.0 ** -0.5
    # decode selection policies (m12_runtime.py:98-166 fields, :1176-1195, :1015-1031)
    decode_relative_a: float | None = None
    decode_relative_max_blocks: int = 48
    decode_relative_union: bool = False
    decode_query_window: int = 1


@dataclass
class M12Oracle:
    """One layer of M12LayerRuntime (m12_runtime.py:169-1346) on numpy arrays.

    Buffers keep the reference's exact content, including the recent window's
    shift-left semantics (m12_runtime.py:1164-1172, :482-503, :777-803) and
    the zero initial contents of sink / recent (m12_runtime.py:200-203).
    All K/V/q arrays hold bf16-representable float32 values.
    """
    cfg: OracleConfig = field(default_factory=OracleConfig)

    def __post_init__(self):
        c = self.cfg
        self.hist_k = np.zeros((0, c.block_size, c.num_kv_heads, c.head_dim), F32)
        self.hist_v = np.zeros_like(self.hist_k)
        self.hist_kq = np.zeros((0, c.block_size, c.num_kv_heads, c.head_dim), np.int8)
        self.hist_vq = np.zeros_like(self.hist_kq)
        self.v_scale = np.zeros((0, c.num_kv_heads), F32)
        self.k_scale = None
        self.reps = np.zeros((c.num_kv_heads, 0, c.r, c.head_dim), F32)
        self.sink_k = np.zeros((c.sink_tokens, c.num_kv_heads, c.head_dim), F32)
        self.sink_v = np.zeros_like(self.sink_k)
        self.recent_k = np.zeros((c.recent_tokens, c.num_kv_heads, c.head_dim), F32)
        self.recent_v = np.zeros_like(self.recent_k)
        self.valid_len = 0
        self.prefill_len = 0
        self.nblocks_filled = 0
        self.protected_blocks: set = set()
        self.last_block_ids = None
        self.pending = None
        self.q_window: list = []   # decode routing queries (m12_runtime.py:1181-1184)

    def reset(self):
        """m12_runtime.py:322-349: lengths cleared, buffers (and their contents) kept."""
        self.nblocks_filled = 0
        self.valid_len = 0
        self.prefill_len = 0
        self.protected_blocks = set()
        self.k_scale = None
        self.last_block_ids = None
        self.pending = None
        self.q_window = []

    # -- store (m12_runtime.py:420-513) ------------------------------------
    def store_kv(self, k, v, with_reps: bool = True):
        """Append a chunk; ``with_reps=False`` leaves reps zero for the caller to fill."""
        c = self.cfg
        k = np.asarray(k, F32)
        v = np.asarray(v, F32)
        T = k.shape[0]
        assert T >= 2
        B = c.block_size
        nb = (T + B - 1) // B
        kp = np.zeros((nb * B,) + k.shape[1:], F32)
        vp = np.zeros_like(kp)
        kp[:T] = k
        vp[:T] = v
        kb = kp.reshape(nb, B, c.num_kv_heads, c.head_dim)
        vb = vp.reshape(nb, B, c.num_kv_heads, c.head_dim)
        start = self.nblocks_filled
        need = start + nb

        def grow(a, n):
            if a.shape[0] < n:
                z = np.zeros((n - a.shape[0],) + a.shape[1:], a.dtype)
                return np.concatenate([a, z])
            return a
        self.hist_k = grow(self.hist_k, need)
        self.hist_v = grow(self.hist_v, need)
        if c.quant_history:
            self.hist_kq = grow(self.hist_kq, need)
            self.hist_vq = grow(self.hist_vq, need)
            self.v_scale = grow(self.v_scale, need)
            if self.k_scale is None:
                self.k_scale = k_scale_from_chunk(kb)
            self.hist_kq[start:need] = quantize(kb, self.k_scale)
            vs = v_scale_per_block(vb)
            self.hist_vq[start:need] = quantize(vb, vs[:, None, :, None])
            self.v_scale[start:need] = vs
        self.hist_k[start:need] = kb
        self.hist_v[start:need] = vb
        if self.reps.shape[1] < need:
            z = np.zeros((c.num_kv_heads, need - self.reps.shape[1], c.r, c.head_dim), F32)
            self.reps = np.concatenate([self.reps, z], axis=1)
        if with_reps:
            self.reps[:, start:need] = build_reps(kb, c.r)[1]
        if self.prefill_len == 0:
            sl = min(c.sink_tokens, T)
            self.sink_k[:sl] = k[:sl]
            self.sink_v[:sl] = v[:sl]
        R = c.recent_tokens
        recent_len = min(R, self.valid_len + T)
        if T >= recent_len:
            self.recent_k[:recent_len] = k[T - recent_len:]
            self.recent_v[:recent_len] = v[T - recent_len:]
        else:
            carry = recent_len - T
            old = min(R, self.valid_len)
            self.recent_k[:carry] = self.recent_k[old - carry:old].copy()
            self.recent_v[:carry] = self.recent_v[old - carry:old].copy()
            self.recent_k[carry:recent_len] = k
            self.recent_v[carry:recent_len] = v
        self.valid_len += T
        self.prefill_len += T
        self.nblocks_filled = need
        self.protected_blocks = protected_blocks_after_store(need, R, B)

    def history_blocks(self, ids):
        """Gathered K/V of the selected blocks as the reference packs them."""
        c = self.cfg
        ids = np.asarray(ids, dtype=np.int64)
        if c.quant_history:
            kq = self.hist_kq[ids].reshape(-1, c.num_kv_heads, c.head_dim)
            vq = self.hist_vq[ids]
            ks = dequant_to_bf16(kq, self.k_scale)
            vs = dequant_to_bf16(vq, self.v_scale[ids][:, None, :, None])
            return ks, vs.reshape(-1, c.num_kv_heads, c.head_dim)
        return (self.hist_k[ids].reshape(-1, c.num_kv_heads, c.head_dim),
                self.hist_v[ids].reshape(-1, c.num_kv_heads, c.head_dim))

    def select(self, q, budget=None):
        c = self.cfg
        req = c.top_k_blocks if budget is None else budget
        return select_blocks(q, self.reps, self.nblocks_filled, c.num_kv_heads,
                             self.protected_blocks, req)

    # -- prefill (m12_runtime.py:518-651) ----------------------------------
    def prefill_first(self, q, k, v):
        assert self.prefill_len == 0
        self.store_kv(k, v)

    def _pack_prior(self, ids):
        """[selected | sink | previous recent] for chunk/verify (m12_runtime.py:560-636)."""
        c = self.cfg
        hk, hv = self.history_blocks(ids)
        sink_len = min(c.sink_tokens, self.valid_len)
        _, off, ln = prefill_recent_slice(self.valid_len, c.sink_tokens, c.recent_tokens)
        pk = np.concatenate([hk, self.sink_k[:sink_len], self.recent_k[off:off + ln]])
        pv = np.concatenate([hv, self.sink_v[:sink_len], self.recent_v[off:off + ln]])
        return pk, pv, hk.shape[0]

    def prefill_chunk(self, q, k, v):
        c = self.cfg
        assert self.prefill_len > 0
        qs = query_summaries(q, c.prefill_query_segments)
        ids, _ = self.select(qs, c.prefill_top_k_blocks)
        pk, pv, _ = self._pack_prior(ids)
        off = pk.shape[0]
        pk = np.concatenate([pk, np.asarray(k, F32)])
        pv = np.concatenate([pv, np.asarray(v, F32)])
        mask = causal_mask(q.shape[0], pk.shape[0], off)
        o = attention_fp64(q, pk, pv, c.scale, mask)
        self.store_kv(k, v)
        self.last_block_ids = ids
        return ids, o

    def prefill_chunk_tiled(self, q, k, v, tile: int):
        """prefill_chunk with one selection per tile of `tile` queries.

        No reference counterpart: the reference selects once per chunk from
        its query summary (m12_runtime.py:550-556); here that routing is
        applied to each tile -- tile i's summary is the bf16 mean of queries
        [i*tile, min(T, (i+1)*tile)) (query_summaries with one segment), its
        Top-K uses the chunk's protected set and budget, and its queries
        attend [its blocks | sink | previous recent | chunk (causal)] as
        prefill_chunk's do.  Returns (ids [ntiles, K], o [T, Hq, D])."""
        c = self.cfg
        assert self.prefill_len > 0
        q = np.asarray(q, F32)
        kc, vc = np.asarray(k, F32), np.asarray(v, F32)
        T = q.shape[0]
        all_ids, outs = [], []
        for t0 in range(0, T, tile):
            t1 = min(T, t0 + tile)
            ids, _ = self.select(query_summaries(q[t0:t1], 1), c.prefill_top_k_blocks)
            pk, pv, _ = self._pack_prior(ids)
            off = pk.shape[0]
            pk = np.concatenate([pk, kc])
            pv = np.concatenate([pv, vc])
            mask = causal_mask(T, pk.shape[0], off)[t0:t1]
            outs.append(attention_fp64(q[t0:t1], pk, pv, c.scale, mask))
            all_ids.append(ids)
        self.store_kv(k, v)
        ids = np.stack(all_ids)
        self.last_block_ids = ids
        return ids, np.concatenate(outs)

    # -- decode (m12_runtime.py:1141-1346) ---------------------------------
    def route_query(self, q0):
        """Decode routing query (m12_runtime.py:1176-1189): with a window W > 1
        the current query joins the last W queries and the route is their
        mean (the current query alone while the window holds one); attention
        still uses the current query.  q0: [Hq, D]."""
        W = self.cfg.decode_query_window
        if W <= 1:
            return q0
        self.q_window.append(np.array(q0, F32))
        del self.q_window[:-W]
        if len(self.q_window) == 1:
            return self.q_window[0]
        return query_summaries(np.stack(self.q_window), 1)[0]

    def decode(self, q, k, v, budget=None):
        c = self.cfg
        q = np.asarray(q, F32)
        assert q.shape[0] == 1
        self.recent_k[:-1] = self.recent_k[1:].copy()
        self.recent_v[:-1] = self.recent_v[1:].copy()
        self.recent_k[-1] = np.asarray(k, F32)[0]
        self.recent_v[-1] = np.asarray(v, F32)[0]
        q_route = self.route_query(q[0])
        req = c.top_k_blocks if (budget is None and c.decode_top_k_blocks is None) else (
            c.decode_top_k_blocks if budget is None else budget)
        if c.decode_relative_a is not None:
            scores = block_scores(q_route[None], self.reps, self.nblocks_filled, c.num_kv_heads)
            ids, vals = relative_threshold_select(scores, self.protected_blocks, req, c.decode_relative_a,
                                                  c.scale, c.decode_relative_max_blocks,
                                                  c.decode_relative_union)
        else:
            ids, vals = self.select(q_route, req)
        hk, hv = self.history_blocks(ids)
        sink_len = min(c.sink_tokens, self.valid_len)
        recent_len = min(c.recent_tokens, self.valid_len + 1)
        pk = np.concatenate([hk, self.sink_k[:sink_len], self.recent_k[c.recent_tokens - recent_len:]])
        pv = np.concatenate([hv, self.sink_v[:sink_len], self.recent_v[c.recent_tokens - recent_len:]])
        o = attention_fp64(q, pk, pv, c.scale)
        self.valid_len += 1
        self.last_block_ids = ids
        return ids, vals, o

    # -- verify (m12_runtime.py:656-807) ------------------------------------
    def verify_tokens(self, q, k, v, lossless=False):
        c = self.cfg
        q = np.asarray(q, F32)
        tq = q.shape[0]
        if lossless:
            ids, allowed, _ = select_per_query(q, self.reps, self.nblocks_filled, c.num_kv_heads,
                                               self.protected_blocks, c.top_k_blocks)
        else:
            ids, _ = self.select(q)
        pk, pv, sel_tokens = self._pack_prior(ids)
        off = pk.shape[0]
        pk = np.concatenate([pk, np.asarray(k, F32)])
        pv = np.concatenate([pv, np.asarray(v, F32)])
        attn_mask = lossless_history_mask(allowed, c.block_size, pk.shape[0]) if lossless else None
        mask = causal_mask(tq, pk.shape[0], off, attn_mask)
        o = attention_fp64(q, pk, pv, c.scale, mask)
        self.pending = (np.asarray(k, F32), np.asarray(v, F32))
        self.last_block_ids = ids
        return ids, o

    def commit_verified(self, n: int):
        """m12_runtime.py:777-803."""
        if n <= 0:
            self.pending = None
            return
        k, v = self.pending[0][:n], self.pending[1][:n]
        T = int(n)
        R = self.cfg.recent_tokens
        old = min(R, self.valid_len)
        new = min(R, self.valid_len + T)
        if T >= R:
            self.recent_k[:R] = k[-R:]
            self.recent_v[:R] = v[-R:]
        else:
            carry = new - T
            if carry > 0:
                self.recent_k[:carry] = self.recent_k[old - carry:old].copy()
                self.recent_v[:carry] = self.recent_v[old - carry:old].copy()
            self.recent_k[carry:carry + T] = k
            self.recent_v[carry:carry + T] = v
        self.valid_len += T
        self.pending = None

    def rollback_verified(self):
        self.pending = None
