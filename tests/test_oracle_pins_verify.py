"""Pins of the oracle's lossless verify mask, int8 history dequantisation and
decode query window (oracle/nkv_oracle.py) -- CPU only.

Every check here is a hand-derived known answer: tiny configurations whose
keys are all zero (so every visible key gets the same softmax weight) and
whose values are one-hot tags e_t, so the attention output of a query reads
back exactly which tokens it attended, with multiplicity:
o = (sum of e_t over the attended keys) / (number of attended keys).
Selection is steered by hand-set representatives: block b's single
representative is the unit vector on dimension 20 + b, and a query with
weight w on that dimension scores w on block b.

Each group ends with planted mistakes (each a plausible slip in the oracle:
the negation dropped, the block flags tiled instead of repeated, the scale
broadcast on the wrong axis, the window never trimmed ...) patched into the
oracle for the duration of one test, and the known answers must fail on
every one of them.
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O

F32 = np.float32
D = 32


def _cfg(**kw):
    base = dict(block_size=2, r=1, recent_tokens=4, sink_tokens=2, top_k_blocks=1,
                num_heads=2, num_kv_heads=1, head_dim=D, scale=1.0)
    base.update(kw)
    return O.OracleConfig(**base)


def _zero_k_tagged_v(tags):
    k = np.zeros((len(tags), 1, D), F32)
    v = np.zeros_like(k)
    for i, t in enumerate(tags):
        v[i, 0, t] = 1.0
    return k, v


def _steered_oracle(**kw):
    """12 prefill tokens tagged 1..12 in blocks b0 = [1, 2] ... b5 = [11, 12].
    Protected: {0} | [6 - 4/2, 6) = {0, 4, 5}; selectable 1, 2, 3.
    Sink [1, 2]; recent window [9, 10, 11, 12]; prefill_recent_slice(12, 2, 4)
    = (8, 0, 4): the whole window follows the sink."""
    ob = O.M12Oracle(_cfg(**kw))
    ob.store_kv(*_zero_k_tagged_v(range(1, 13)))
    assert ob.protected_blocks == {0, 4, 5}
    reps = np.zeros_like(ob.reps)
    for b in (1, 2, 3):
        reps[0, b, 0, 20 + b] = 1.0
    ob.reps = reps
    return ob


def _query(weights):
    """One query [Hq=2, D]: weight w on dimension 20 + b for each {b: w}."""
    q = np.zeros((2, D), F32)
    for b, w in weights.items():
        q[:, 20 + b] = w
    return q


def _mean_of_tags(tags):
    want = np.zeros(D)
    for t in tags:
        want[t] += 1.0 / len(tags)
    return want


BLOCK_TAGS = {1: [3, 4], 2: [5, 6], 3: [7, 8]}
SINK = [1, 2]
RECENT = [9, 10, 11, 12]
CHUNK = [13, 14, 15]


def _expected_verify(blocks_per_query):
    """Query t reads its blocks' tokens, the sink, the whole recent window and
    chunk tokens 13 .. 13 + t (causal, m12_runtime.py:877-883)."""
    out = []
    for t, blocks in enumerate(blocks_per_query):
        tags = [x for b in blocks for x in BLOCK_TAGS[b]] + SINK + RECENT + CHUNK[:t + 1]
        out.append(_mean_of_tags(tags))
    return out


# ---- lossless verify: per-query mask over the union (m12_runtime.py:677-680, :746-758) ------------

VERIFY_CASES = [
    # (top_k, query weights, expected union, blocks each query may read, shared-mode blocks)
    # budget 1, each query steered to a different block; shared = the max over queries (b2: 2)
    (1, [{2: 2.0}, {1: 1.0}, {3: 1.5}], [1, 2, 3], [[2], [1], [3]], [2]),
    # budget 2, overlapping selections: every pair of blocks once
    (2, [{1: 2.0, 2: 1.0}, {2: 1.0, 3: 2.0}, {3: 1.0, 1: 0.5}], [1, 2, 3],
     [[1, 2], [2, 3], [1, 3]], [1, 3]),
    # a gap in the union (block 2 unused): union columns are blocks 1 and 3
    (1, [{3: 2.0}, {1: 1.0}, {3: 0.5}], [1, 3], [[3], [1], [3]], [3]),
]


def _check_verify_known_answers():
    for top_k, weights, union, per_query, shared in VERIFY_CASES:
        q = np.stack([_query(w) for w in weights])
        kc, vc = _zero_k_tagged_v(CHUNK)
        # lossless: union of per-query selections, each query masked to its own blocks
        ob = _steered_oracle(top_k_blocks=top_k)
        ids, o = ob.verify_tokens(q, kc, vc, lossless=True)
        assert ids.tolist() == union
        for t, want in enumerate(_expected_verify(per_query)):
            for h in range(2):
                assert np.allclose(o[t, h], want, rtol=0, atol=1e-12), (top_k, t, h)
        # shared: one selection, the max over the queries, read by every query
        ob = _steered_oracle(top_k_blocks=top_k)
        ids, o = ob.verify_tokens(q, kc, vc, lossless=False)
        assert ids.tolist() == shared
        for t, want in enumerate(_expected_verify([shared] * 3)):
            assert np.allclose(o[t, 0], want, rtol=0, atol=1e-12), (top_k, t)
        # the verify pass leaves the store untouched until commit
        assert ob.valid_len == 12 and ob.pending is not None


def test_verify_lossless_and_shared_known_answers():
    _check_verify_known_answers()


def test_lossless_mask_small_literal():
    """Two queries, union of 3 blocks of 2 keys, 10 packed keys: the flags
    repeat per key of each block, negated; keys 6..9 stay unmasked."""
    allowed = np.array([[True, False, True], [False, True, False]])
    m = O.lossless_history_mask(allowed, 2, 10)
    assert m.astype(int).tolist() == [[0, 0, 1, 1, 0, 0, 0, 0, 0, 0],
                                      [1, 1, 0, 0, 1, 1, 0, 0, 0, 0]]


def _mask_no_negation(allowed, block_size, s_len):
    m = np.zeros((allowed.shape[0], s_len), bool)
    m[:, :allowed.shape[1] * block_size] = np.repeat(allowed, block_size, axis=1)
    return m


def _mask_tiled(allowed, block_size, s_len):
    m = np.zeros((allowed.shape[0], s_len), bool)
    m[:, :allowed.shape[1] * block_size] = ~np.tile(allowed, (1, block_size))
    return m


def _mask_wrong_repeat_axis(allowed, block_size, s_len):
    m = np.zeros((allowed.shape[0], s_len), bool)
    m[:, :allowed.shape[1] * block_size] = ~np.repeat(allowed, block_size, axis=0)
    return m


def _mask_hides_sink_and_recent(allowed, block_size, s_len):
    m = np.zeros((allowed.shape[0], s_len), bool)
    u = allowed.shape[1] * block_size
    m[:, :u] = ~np.repeat(allowed, block_size, axis=1)
    m[:, u:s_len - allowed.shape[0]] = True
    return m


@pytest.mark.parametrize("wrong", [_mask_no_negation, _mask_tiled, _mask_wrong_repeat_axis,
                                   _mask_hides_sink_and_recent])
def test_verify_pins_fail_on_planted_mask_mistakes(monkeypatch, wrong):
    monkeypatch.setattr(O, "lossless_history_mask", wrong)
    with pytest.raises((AssertionError, ValueError)):
        _check_verify_known_answers()


# ---- int8 history gather + dequant (m12_runtime.py:1262-1267, fused_dequant.py:24-44) ------------

KS = np.array([[1, 2, 4, 8], [0.5, 0.25, 0.125, 16]], F32)           # k_scale [Hkv, D]
VS = np.array([[1, 2], [3, 5], [0.75, 1.5]], F32)                     # v_scale [block, Hkv]


def _int8_oracle():
    """3 blocks of 2 tokens, Hkv = 2, D = 4, codes set by hand:
    K code(b, i, h, d) = s_i ((b + 1)(d + 1) + 10 h), V code(b, i, h, d) =
    s_i (d + 1 + 4 h), with s_0 = +1, s_1 = -1 (token i of the block)."""
    ob = O.M12Oracle(O.OracleConfig(block_size=2, r=1, recent_tokens=4, sink_tokens=2, num_heads=4,
                                    num_kv_heads=2, head_dim=4, quant_history=True))
    kq = np.zeros((3, 2, 2, 4), np.int8)
    vq = np.zeros_like(kq)
    for b in range(3):
        for i, s in enumerate((1, -1)):
            for h in range(2):
                for d in range(4):
                    kq[b, i, h, d] = s * ((b + 1) * (d + 1) + 10 * h)
                    vq[b, i, h, d] = s * (d + 1 + 4 * h)
    ob.hist_kq, ob.hist_vq, ob.k_scale, ob.v_scale = kq, vq, KS.copy(), VS.copy()
    ob.nblocks_filled = 3
    return ob


# ids [2, 0]: rows b2 token 0, b2 token 1, b0 token 0, b0 token 1 -- worked by hand:
# K b2 h0 codes 3, 6, 9, 12 x (1, 2, 4, 8); h1 codes 13, 16, 19, 22 x (0.5, 0.25, 0.125, 16)
# K b0 h0 codes 1, 2, 3, 4 x (1, 2, 4, 8);  h1 codes 11, 12, 13, 14 x (...)
# V codes h0 1, 2, 3, 4; h1 5, 6, 7, 8, times v_scale[block, h]: b2 (0.75, 1.5), b0 (1, 2)
WANT_K = [[[3, 12, 36, 96], [6.5, 4, 2.375, 352]],
          [[-3, -12, -36, -96], [-6.5, -4, -2.375, -352]],
          [[1, 4, 12, 32], [5.5, 3, 1.625, 224]],
          [[-1, -4, -12, -32], [-5.5, -3, -1.625, -224]]]
WANT_V = [[[0.75, 1.5, 2.25, 3], [7.5, 9, 10.5, 12]],
          [[-0.75, -1.5, -2.25, -3], [-7.5, -9, -10.5, -12]],
          [[1, 2, 3, 4], [10, 12, 14, 16]],
          [[-1, -2, -3, -4], [-10, -12, -14, -16]]]


def _reference_torch_dequant(ob, ids):
    """The reference's eager op sequence on flattened token rows
    (m12_runtime.py:1262-1267): K = (codes.float() * k_scale).to(bf16);
    row_scale = v_scale[ids].repeat_interleave(B, dim=0);
    V = (codes.float() * row_scale[:, :, None]).to(bf16)."""
    B = ob.cfg.block_size
    idx = torch.as_tensor(np.asarray(ids, np.int64))
    kq = torch.from_numpy(ob.hist_kq)[idx].reshape(-1, ob.cfg.num_kv_heads, ob.cfg.head_dim)
    vq = torch.from_numpy(ob.hist_vq)[idx].reshape(-1, ob.cfg.num_kv_heads, ob.cfg.head_dim)
    k = (kq.float() * torch.from_numpy(ob.k_scale)).to(torch.bfloat16).float().numpy()
    row_scale = torch.from_numpy(ob.v_scale)[idx].repeat_interleave(B, dim=0)
    v = (vq.float() * row_scale[:, :, None]).to(torch.bfloat16).float().numpy()
    return k, v


def _check_int8_known_answers():
    ob = _int8_oracle()
    k, v = ob.history_blocks([2, 0])
    assert k.tolist() == WANT_K
    assert v.tolist() == WANT_V
    # rounding point: random codes and inexact scales against the reference's torch sequence
    rng = np.random.default_rng(7)
    kb = O.bf16_round(rng.standard_normal((9, 64, 8, 128)).astype(F32) * 0.3)
    vb = O.bf16_round(rng.standard_normal((9, 64, 8, 128)).astype(F32) * 0.3)
    ob = O.M12Oracle(O.OracleConfig(quant_history=True))
    ob.store_kv(kb.reshape(-1, 8, 128), vb.reshape(-1, 8, 128), with_reps=False)
    for ids in ([7, 2, 5], [0, 8, 1, 3]):
        k, v = ob.history_blocks(ids)
        rk, rv = _reference_torch_dequant(ob, ids)
        assert np.array_equal(k, rk) and np.array_equal(v, rv)


def test_int8_history_blocks_known_answers():
    _check_int8_known_answers()


def _history_blocks_scale_by_position(self, ids):
    c = self.cfg
    ids = np.asarray(ids, dtype=np.int64)
    kq = self.hist_kq[ids].reshape(-1, c.num_kv_heads, c.head_dim)
    ks = O.dequant_to_bf16(kq, self.k_scale)
    vs = O.dequant_to_bf16(self.hist_vq[ids], self.v_scale[:len(ids)][:, None, :, None])
    return ks, vs.reshape(-1, c.num_kv_heads, c.head_dim)


def _history_blocks_v_scale_wrong_axis(self, ids):
    c = self.cfg
    ids = np.asarray(ids, dtype=np.int64)
    kq = self.hist_kq[ids].reshape(-1, c.num_kv_heads, c.head_dim)
    ks = O.dequant_to_bf16(kq, self.k_scale)
    vs = O.dequant_to_bf16(self.hist_vq[ids], self.v_scale[ids][:, :, None, None])
    return ks, vs.reshape(-1, c.num_kv_heads, c.head_dim)


def _history_blocks_truncating(self, ids):
    c = self.cfg
    ids = np.asarray(ids, dtype=np.int64)
    kq = self.hist_kq[ids].reshape(-1, c.num_kv_heads, c.head_dim).astype(F32)
    vq = self.hist_vq[ids].astype(F32)

    def trunc(x):
        return (np.asarray(x, F32).view(np.uint32) & np.uint32(0xFFFF0000)).view(F32)
    ks = trunc(kq * self.k_scale)
    vs = trunc(vq * self.v_scale[ids][:, None, :, None])
    return ks, vs.reshape(-1, c.num_kv_heads, c.head_dim)


@pytest.mark.parametrize("wrong", [_history_blocks_scale_by_position, _history_blocks_v_scale_wrong_axis,
                                   _history_blocks_truncating])
def test_int8_pins_fail_on_planted_mistakes(monkeypatch, wrong):
    monkeypatch.setattr(O.M12Oracle, "history_blocks", wrong)
    with pytest.raises((AssertionError, ValueError)):
        _check_int8_known_answers()


# ---- decode query window (m12_runtime.py:1176-1189, reset :340) ------------------------------------

# step: current query weights -> the window after the step -> the routed block
#  1  3 e21             [3 e21]                   the window holds one query: route = q -> b1
#  2  2 e22             [3 e21, 2 e22]            mean 1.5 e21 + 1 e22 -> b1 (q alone: b2)
#  3  4 e22             [3 e21, 2 e22, 4 e22]     mean 1 e21 + 2 e22 -> b2
#  4  5 e21             [2 e22, 4 e22, 5 e21]     mean 5/3 e21 + 2 e22 -> b2 (untrimmed: 2 e21 + 1.5 e22 -> b1)
#  5  7 e21             [4 e22, 5 e21, 7 e21]     mean 4 e21 + 4/3 e22 -> b1
# after reset + a new prefill: 2 e22 alone -> b2 (a stale window would route to b1)
WINDOW_STEPS = [({1: 3.0}, 1), ({2: 2.0}, 1), ({2: 4.0}, 2), ({1: 5.0}, 2), ({1: 7.0}, 1)]


def _decode_window_step(ob, weights, tag):
    k, v = _zero_k_tagged_v([tag])
    ids, _, o = ob.decode(_query(weights)[None], k, v)
    return ids.tolist(), o[0, 0]


def _check_window_known_answers():
    ob = _steered_oracle(decode_query_window=3)
    recent = list(RECENT)
    for step, (weights, block) in enumerate(WINDOW_STEPS):
        tag = 16 + step
        ids, o = _decode_window_step(ob, weights, tag)
        assert ids == [block], (step, ids)
        recent = recent[1:] + [tag]
        # attends its routed block, the sink and the shifted recent window (new token last)
        assert np.allclose(o, _mean_of_tags(BLOCK_TAGS[block] + SINK + recent), rtol=0, atol=1e-12)
    ob.reset()
    ob.store_kv(*_zero_k_tagged_v(range(1, 13)))
    reps = np.zeros_like(ob.reps)
    for b in (1, 2, 3):
        reps[0, b, 0, 20 + b] = 1.0
    ob.reps = reps
    ids, _ = _decode_window_step(ob, {2: 2.0}, 30)
    assert ids == [2]


def test_decode_query_window_known_answers():
    _check_window_known_answers()


def test_decode_query_window_of_one_routes_the_current_query():
    ob = _steered_oracle(decode_query_window=1)
    got = [_decode_window_step(ob, w, 16 + i)[0][0] for i, (w, _) in enumerate(WINDOW_STEPS)]
    assert got == [1, 2, 2, 1, 1]


def _route_untrimmed(self, q0):
    self.q_window.append(np.array(q0, F32))
    if len(self.q_window) == 1:
        return self.q_window[0]
    return O.query_summaries(np.stack(self.q_window), 1)[0]


def _route_current_only(self, q0):
    return q0


def _route_previous_queries(self, q0):
    W = self.cfg.decode_query_window
    prev = list(self.q_window)
    self.q_window.append(np.array(q0, F32))
    del self.q_window[:-W]
    if not prev:
        return q0
    return O.query_summaries(np.stack(prev[-W:]), 1)[0]


_ORIGINAL_RESET = O.M12Oracle.reset


def _reset_keeping_window(self):
    kept = list(self.q_window)
    _ORIGINAL_RESET(self)
    self.q_window = kept


@pytest.mark.parametrize("attr,wrong", [("route_query", _route_untrimmed),
                                        ("route_query", _route_current_only),
                                        ("route_query", _route_previous_queries),
                                        ("reset", _reset_keeping_window)])
def test_window_pins_fail_on_planted_mistakes(monkeypatch, attr, wrong):
    monkeypatch.setattr(O.M12Oracle, attr, wrong)
    with pytest.raises(AssertionError):
        _check_window_known_answers()
