"""Pins of the CPU oracle (oracle/nkv_oracle.py) -- no GPU needed.

Each oracle function is checked against (a) the known answers the
reference's own tests hold, (b) an independent formulation that mathematics
fixes (exact rational arithmetic, brute force, textbook softmax), chosen so
that a dropped term, a swapped operand or a wrong index fails.
"""

import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O


# ---------------------------------------------------------------- rounding --

def test_bf16_round_matches_torch_and_ties_to_even():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(10000) * np.exp(rng.uniform(-20, 20, 10000))).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(x), ref)
    # exact halfway cases: 1 + 2^-8 lies between 1 and 1 + 2^-7 -> even (1.0)
    half = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)], dtype=np.float32)
    assert O.bf16_round(half).tolist() == [1.0, 1 + 2 ** -6, -1.0]


def test_f64_to_bf16_is_one_correct_rounding():
    rng = random.Random(1)
    for _ in range(3000):
        v = rng.uniform(-1, 1) * 2.0 ** rng.randint(-140, 100)
        got = float(O.f64_to_bf16(np.array([v]))[0])
        # exact: the bf16 grid around v, nearest, ties to even (Fraction arithmetic)
        fv = Fraction(v)
        m, e = math.frexp(v)
        q = Fraction(2) ** max(e - 8, -133)          # bf16 quantum at this binade
        lo = (fv / q).__floor__()
        cands = [lo * q, (lo + 1) * q]
        d0, d1 = abs(fv - cands[0]), abs(fv - cands[1])
        if d0 < d1 or (d0 == d1 and lo % 2 == 0):
            want = cands[0]
        else:
            want = cands[1]
        assert Fraction(got) == want, v


# ----------------------------------------------------------------- scores --

def _rand_bf16(rng, shape, scale=1.0):
    return O.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def test_block_scores_equal_a_pure_python_sequential_loop():
    rng = np.random.default_rng(2)
    q = _rand_bf16(rng, (2, 8, 128))          # Nq=2, Hq=8
    reps = _rand_bf16(rng, (2, 5, 3, 128), 128 ** -0.5)   # Hkv=2, nb=5, r=3
    got = O.block_scores(q, reps, 5, 2)
    for b in range(5):
        best = None
        for n in range(2):
            for hq in range(8):
                h = hq // 4
                for j in range(3):
                    acc = np.float32(0.0)
                    for d in range(128):
                        acc = np.float32(acc + np.float32(q[n, hq, d]) * np.float32(reps[h, b, j, d]))
                    best = acc if best is None else max(best, acc)
        assert np.float32(got[b]) == best


def test_block_scores_are_the_exact_dot_within_fp32_bound():
    rng = np.random.default_rng(3)
    q = _rand_bf16(rng, (1, 32, 128))
    reps = _rand_bf16(rng, (8, 6, 4, 128), 128 ** -0.5)
    got = O.block_scores(q, reps, 6, 8)
    u = 2.0 ** -24
    for b in range(6):
        exact_best, bound = None, 0.0
        for hq in range(32):
            h = hq // 4
            for j in range(4):
                terms = [Fraction(float(q[0, hq, d])) * Fraction(float(reps[h, b, j, d])) for d in range(128)]
                ex = sum(terms, Fraction(0))
                if exact_best is None or ex > exact_best:
                    exact_best = ex
                bound = max(bound, 128 * u * float(sum(abs(t) for t in terms)))
        assert abs(Fraction(float(got[b])) - exact_best) <= Fraction(bound)


def test_gqa_map_routes_each_query_head_to_its_kv_head():
    # block_sparse.py:33-41 / test_block_sparse.py:192-207: heads 0..3 -> kv 0, 4..7 -> kv 1
    assert O.kv_head_for_query(4, 2).tolist() == [0, 0, 1, 1]
    reps = np.zeros((2, 2, 1, 128), np.float32)
    reps[1, 1, 0, 0] = 1.0            # only KV head 1, block 1 has signal
    q = np.zeros((1, 8, 128), np.float32)
    q[0, 5, 0] = 2.0                  # query head 5 -> KV head 1: sees it
    assert O.block_scores(q, reps, 2, 2).tolist() == [0.0, 2.0]
    q[0, 5, 0] = 0.0
    q[0, 2, 0] = 2.0                  # query head 2 -> KV head 0: does not
    assert O.block_scores(q, reps, 2, 2).tolist() == [0.0, 0.0]


# ------------------------------------------------------------------ top-k --

def test_topk_known_answers_from_reference_tests():
    # test_block_sparse.py:156-161
    ids, vals = O.topk_blocks(np.array([0.0, 5.0, 1.0, 4.0, 2.0], np.float32), set(), 2)
    assert ids.tolist() == [1, 3] and vals.tolist() == [5.0, 4.0]
    # test_m19_selector_graph.py:68-87: budget capped after protection; all protected -> one id
    s = np.array([0.3, 0.1, 0.2], np.float32)
    ids, _ = O.topk_blocks(s, {0, 20}, 6)
    assert ids.tolist() == [2, 1]
    ids, _ = O.topk_blocks(s, {0, 1, 2, 20}, 6)
    assert ids.tolist() == [0]
    # test_m21_static_mask.py:28-45: exact ties, protected {0, 4}
    ids, _ = O.topk_blocks(np.zeros(8, np.float32), {0, 4, 100}, 6)
    assert ids.tolist() == [1, 2, 3, 5, 6, 7]


def test_topk_against_brute_force_sort():
    rng = random.Random(4)
    for _ in range(300):
        nb = rng.randint(1, 40)
        s = np.array([rng.choice([rng.uniform(-3, 3), 0.5, -0.0, float("-inf")]) for _ in range(nb)], np.float32)
        prot = {rng.randint(-2, nb + 2) for _ in range(rng.randint(0, 5))}
        k = rng.randint(1, 45)
        ids, vals = O.topk_blocks(s, prot, k)
        masked = [(-math.inf if b in prot else float(s[b])) for b in range(nb)]
        n_prot = len([p for p in prot if 0 <= p < nb])
        kk = min(k, max(1, nb - n_prot))
        want = sorted(range(nb), key=lambda b: (-masked[b], b))[:kk]
        assert ids.tolist() == want


def test_per_query_union_and_allowed_mask():
    rng = np.random.default_rng(5)
    q = _rand_bf16(rng, (3, 8, 128))
    reps = _rand_bf16(rng, (2, 20, 2, 128), 128 ** -0.5)
    prot = {0, 19}
    union, allowed, tops = O.select_per_query(q, reps, 20, 2, prot, 4)
    for t in range(3):
        own = O.topk_blocks(O.block_scores(q[t:t + 1], reps, 20, 2), prot, 4)[0]
        assert tops[t].tolist() == own.tolist()
        assert set(union[allowed[t]].tolist()) == set(own.tolist())
    assert union.tolist() == sorted(set(tops.reshape(-1).tolist()))


def test_dynamic_top_k_known_answers():
    # test_m16_dynamic_topk.py:13-22
    f = O.dynamic_top_k_from_scores
    assert f(np.ones(32, np.float32), 32, 0.90) == 32
    assert f(np.arange(10, 0, -1).astype(np.float32), 32, 0.90) == 10
    assert f(np.array([np.inf] + [0.0] * 31, np.float32), 32, 0.90) == 32
    assert f(np.array([10.0] + [0.0] * 31, np.float32), 32, 0.90) == 16


# ------------------------------------------------------------ bookkeeping --

def test_prefill_recent_slice_known_answers():
    # test_m14_prefill_layout.py:34-44
    assert O.prefill_recent_slice(4096, 64, 512) == (3584, 0, 512)
    assert O.prefill_recent_slice(128, 64, 512) == (0, 64, 64)
    assert O.prefill_recent_slice(64, 64, 512) == (0, 64, 0)


def test_prefill_layout_covers_every_prior_token_once():
    # test_m14_prefill_layout.py:12-37: selected (all non-protected) + sink + recent
    valid_len, B, S, R = 4096, 64, 64, 512
    nb = valid_len // B
    prot = O.protected_blocks_after_store(nb, R, B)
    selected = {t for b in range(nb) if b not in prot for t in range(b * B, (b + 1) * B)}
    sink = set(range(min(S, valid_len)))
    start, off, ln = O.prefill_recent_slice(valid_len, S, R)
    recent = set(range(start + off, start + off + ln))
    assert not (selected & sink) and not (selected & recent) and not (sink & recent)
    assert selected | sink | recent == set(range(valid_len))


def test_protected_set_after_store():
    # m12_runtime.py:509-513: {0} U last 8 blocks
    assert O.protected_blocks_after_store(128, 512, 64) == {0} | set(range(120, 128))
    assert O.protected_blocks_after_store(5, 512, 64) == {0, 1, 2, 3, 4}


def test_query_summaries_are_segment_means():
    # test_m14_prefill_layout.py:47-58 (values exact in bf16)
    q = np.arange(8 * 2 * 3, dtype=np.float32).reshape(8, 2, 3)
    assert np.array_equal(O.query_summaries(q, 1)[0], q.mean(axis=0))
    want = np.stack([q[0:2].mean(0), q[2:4].mean(0), q[4:6].mean(0), q[6:8].mean(0)])
    assert np.array_equal(O.query_summaries(q, 4), want)
    # tensor_split bounds with a remainder: 10 tokens in 4 parts -> 3, 3, 2, 2
    assert O.tensor_split_bounds(10, 4) == [(0, 3), (3, 6), (6, 8), (8, 10)]
    assert [t.shape[0] for t in torch.tensor_split(torch.zeros(10), 4)] == [3, 3, 2, 2]


# -------------------------------------------------------------- attention --

def test_attention_matches_manual_softmax():
    # test_block_sparse.py:36-49: per-head manual softmax(q k^T / sqrt(d)) v
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 4, 8))
    k = rng.standard_normal((10, 2, 8))
    v = rng.standard_normal((10, 2, 8))
    out = O.attention_fp64(q, k, v, 8 ** -0.5)
    for hq in range(4):
        h = hq // 2
        logits = [sum(q[0, hq, d] * k[s, h, d] for d in range(8)) * 8 ** -0.5 for s in range(10)]
        mx = max(logits)
        w = [math.exp(x - mx) for x in logits]
        tot = sum(w)
        for d in range(8):
            want = sum(w[s] / tot * v[s, h, d] for s in range(10))
            assert abs(out[0, hq, d] - want) < 1e-12


def test_causal_mask_and_select_all_equals_dense():
    # m12_runtime.py:877-883: query t sees history and chunk keys <= t
    m = O.causal_mask(3, 6, 3)
    assert m.tolist() == [[False, False, False, False, True, True],
                          [False, False, False, False, False, True],
                          [False, False, False, False, False, False]]
    # test_block_sparse.py:236-242: attending every token == dense
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 4, 8))
    k = rng.standard_normal((48, 2, 8))
    v = rng.standard_normal((48, 2, 8))
    perm = rng.permutation(48)
    a = O.attention_fp64(q, k, v, 0.3)
    b = O.attention_fp64(q, k[perm], v[perm], 0.3)
    assert np.allclose(a, b, atol=1e-12, rtol=0)


# ------------------------------------------------------------------- int8 --

def test_int8_scheme_matches_torch_round_half_even_and_clamp():
    # quant_kv.py:27-49: round(x / scale).clamp(-127, 127), torch.round = half-to-even
    x = np.array([0.5, 1.5, 2.5, -0.5, -2.5, 300.0, -300.0, 126.5], np.float32)
    assert O.quantize(x, np.float32(1.0)).tolist() == [0, 2, 2, 0, -2, 127, -127, 126]
    rng = np.random.default_rng(8)
    kb = _rand_bf16(rng, (3, 64, 2, 128), 128 ** -0.5)
    ks = O.k_scale_from_chunk(kb)
    t = torch.from_numpy(kb)
    ks_t = t.float().abs().amax(dim=(0, 1)).clamp_min(1e-8) / 127
    assert np.array_equal(ks, ks_t.numpy())
    kq_t = torch.round(t.float() / ks_t).clamp(-127, 127).to(torch.int8)
    assert np.array_equal(O.quantize(kb, ks), kq_t.numpy())
    vs = O.v_scale_per_block(kb)
    vs_t = t.float().abs().amax(dim=(1, 3)).clamp_min(1e-8) / 127
    assert np.array_equal(vs, vs_t.numpy())
    vq_t = torch.round(t.float() / vs_t[:, None, :, None]).clamp(-127, 127).to(torch.int8)
    assert np.array_equal(O.quantize(kb, vs[:, None, :, None]), vq_t.numpy())
    # dequantisation as packed by the reference: bf16(int8 * scale)
    deq_t = (kq_t.float() * ks_t).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.dequant_to_bf16(O.quantize(kb, ks), ks), deq_t)


def test_token_scale_fp16_closed_form():
    x = np.zeros((2, 128), np.float32)
    x[0, 7] = -254.0                      # amax 254 -> 254/127 = 2.0 exactly
    sc = O.token_scale_fp16(x)
    assert sc.dtype == np.float16
    assert float(sc[0]) == 2.0
    assert float(sc[1]) == 2.0 ** -24     # all-zero row: smallest fp16 subnormal


# -------------------------------------------------------- representatives --

def _reps_loop(kb, r):
    """Direct loop restatement of m12_runtime.py:354-395 for one (block, head)."""
    B, D = kb.shape
    dirs = []
    for t in range(B):
        n = math.sqrt(sum(float(x) ** 2 for x in kb[t]))
        dirs.append([float(x) / max(n, 1e-12) for x in kb[t]])
    mean = [sum(dirs[t][d] for t in range(B)) / B for d in range(D)]
    mn = math.sqrt(sum(m * m for m in mean))
    md = [m / max(mn, 1e-12) for m in mean]
    cos0 = [sum(dirs[t][d] * md[d] for d in range(D)) for t in range(B)]
    chosen = [max(range(B), key=lambda t: (cos0[t], -t))]
    for _ in range(1, r):
        def score(t):
            mx = max(sum(dirs[t][d] * dirs[c][d] for d in range(D)) for c in chosen)
            return 2.0 if t in chosen else mx
        chosen.append(min(range(B), key=lambda t: (score(t), t)))
    return chosen


def test_build_reps_matches_loop_restatement_and_invariants():
    rng = np.random.default_rng(9)
    kb = _rand_bf16(rng, (3, 12, 2, 6))           # N=3 blocks, B=12 tokens, Hkv=2, D=6
    kb[2, 5:] = 0.0                               # zero-padded tail of a partial block
    sel, reps, margins = O.build_reps(kb, 4)
    for n in range(3):
        for h in range(2):
            if np.all(margins[n, h] > 1e-9):
                assert sel[n, h].tolist() == _reps_loop(kb[n, :, h], 4)
            assert len(set(sel[n, h].tolist())) == 4          # distinct tokens
            for j in range(4):                                # reps are raw rows of K
                assert np.array_equal(reps[h, n, j], kb[n, sel[n, h, j], h])


# -------------------------------------------------- runtime state machine --

def test_oracle_recent_window_follows_reference_buffer_ops():
    """Decode shift-left + append keeps the last R tokens (m12_runtime.py:1164-1172)."""
    cfg = O.OracleConfig(recent_tokens=128, sink_tokens=64, top_k_blocks=2)
    ob = O.M12Oracle(cfg)
    rng = np.random.default_rng(10)
    T = 640
    k = _rand_bf16(rng, (T, 8, 128), 0.1)
    ob.store_kv(k, k, with_reps=False)
    ob.reps[:] = _rand_bf16(rng, ob.reps.shape, 0.1)
    assert np.array_equal(ob.recent_k, k[T - 128:])
    assert np.array_equal(ob.sink_k, k[:64])
    news = []
    for s in range(5):
        kn = _rand_bf16(rng, (1, 8, 128), 0.1)
        news.append(kn[0])
        ob.decode(_rand_bf16(rng, (1, 32, 128)), kn, kn)
    assert np.array_equal(ob.recent_k, np.concatenate([k[T - 128 + 5:], np.stack(news)]))
    assert ob.valid_len == T + 5


def test_bf16_probability_rounding_sizes_the_prefill_tolerance():
    """Few keys, near-uniform softmax: bf16 P alone moves outputs past one bf16
    ulp of the exact result but stays inside the prefill tolerance."""
    from tests._util import PREFILL_TOL
    rng = np.random.default_rng(5)
    T, S = 90, 254
    q = O.bf16_round(rng.standard_normal((T, 32, 128)).astype(np.float32))
    k = O.bf16_round((0.09 * rng.standard_normal((S, 8, 128))).astype(np.float32))
    v = O.bf16_round((0.09 * rng.standard_normal((S, 8, 128))).astype(np.float32))
    mask = O.causal_mask(T, S, S - T)
    exact = O.attention_fp64(q, k, v, 128 ** -0.5, mask)
    approx = O.bf16_round(O.attention_bf16_probs(q, k, v, 128 ** -0.5, mask).astype(np.float32))
    err = np.abs(approx - exact)
    assert (err > 2.0 ** -7 * np.abs(exact) + 2e-5).any()          # beyond the few-query bound
    assert not (err > PREFILL_TOL["rel"] * np.abs(exact) + PREFILL_TOL["abs_tol"]).any()
    # and with P exact the same comparison is within one bf16 ulp
    assert np.abs(O.bf16_round(exact.astype(np.float32)) - exact).max() <= 2.0 ** -8 * np.abs(exact).max()


# ---- relative-threshold decode selection (m12_runtime.py:1015-1031) --------------

@pytest.mark.parametrize("scores,prot,req,a,scale,cap,union,want", [
    # threshold 5 + ln 0.5 = 4.307: blocks 0 (5.0) and 4 (4.9) pass, in score order
    ([5.0, 4.0, 1.0, 0.0, 4.9], [], 2, 0.5, 1.0, 48, False, [0, 4]),
    # union with the first k = 3 by score adds block 1 (4.0)
    ([5.0, 4.0, 1.0, 0.0, 4.9], [], 3, 0.5, 1.0, 48, True, [0, 4, 1]),
    # block 0 protected: max 4.9, threshold 4.207 keeps block 4 only
    ([5.0, 4.0, 1.0, 0.0, 4.9], [0], 2, 0.5, 1.0, 48, False, [4]),
    # cap 1: only the best candidate can be kept
    ([5.0, 4.0, 1.0, 0.0, 4.9], [], 2, 0.5, 1.0, 1, False, [0]),
    # scale 0.5 doubles the margin: 5 + 2 ln 0.5 = 3.614 also keeps block 1
    ([5.0, 4.0, 1.0, 0.0, 4.9], [], 2, 0.5, 0.5, 48, False, [0, 4, 1]),
    # exact ties pass together, lower ids first
    ([3.0, 3.0, 3.0], [], 1, 0.9, 1.0, 48, False, [0, 1, 2]),
    # every block protected: k = cap = 1 and the -inf threshold keeps block 0
    ([1.0, 2.0, 3.0], [0, 1, 2], 4, 0.5, 1.0, 48, False, [0]),
])
def test_relative_threshold_select_known_answers(scores, prot, req, a, scale, cap, union, want):
    ids, vals = O.relative_threshold_select(np.array(scores, np.float32), prot, req, a, scale, cap, union)
    assert ids.tolist() == want
    s = np.array(scores, np.float32)
    s[prot] = -np.inf
    assert np.array_equal(vals, s[ids])


def test_relative_threshold_matches_brute_force():
    """Random cases against a direct statement: every kept block is within the
    margin and among the first cap by (score desc, id asc); every block within
    the margin among those first cap is kept."""
    rng = np.random.default_rng(3)
    for _ in range(200):
        nb = int(rng.integers(1, 40))
        s = (rng.standard_normal(nb) * 2).astype(np.float32)
        prot = sorted(set(rng.integers(0, nb, int(rng.integers(0, 4))).tolist()))
        a, scale = float(rng.uniform(0.05, 0.95)), float(rng.uniform(0.05, 1.0))
        cap, req = int(rng.integers(1, 20)), int(rng.integers(1, 20))
        ids, _ = O.relative_threshold_select(s, prot, req, a, scale, cap, False)
        sm = s.copy()
        sm[prot] = -np.inf
        ranked = sorted(range(nb), key=lambda b: (-float(sm[b]), b))
        avail = nb - len(prot)
        first = ranked[:min(cap, max(1, avail))]
        thr = np.float32(float(sm.max()) + np.log(a) / scale)
        within = [b for b in first if sm[b] >= thr]
        k = min(req, max(1, avail))
        assert ids.tolist() == (within if within else ranked[:k])


# ---- recent window: carry, commit and short-history decode -------------------------
#
# Token t (1-based) is tagged by the value t in every K dimension and by the
# one-hot vector e_t in V, so buffer contents read back as token ids (0 = a
# slot never written) and, with q = 0, the attention output is the mean of
# the attended one-hot rows: o[t] = (times token t is attended) / (keys).

def _tiny_cfg(R=4, S=2):
    return O.OracleConfig(block_size=2, r=1, recent_tokens=R, sink_tokens=S, top_k_blocks=1,
                          num_heads=2, num_kv_heads=1, head_dim=16, scale=1.0)


def _tagged(ids):
    ids = list(ids)
    k = np.zeros((len(ids), 1, 16), np.float32)
    v = np.zeros_like(k)
    for i, t in enumerate(ids):
        k[i, 0, :] = t
        v[i, 0, t] = 1.0
    return k, v


def _recent_tags(ob):
    return ob.recent_k[:, 0, 0].astype(int).tolist()


def _decode_tagged(ob, t):
    k, v = _tagged([t])
    _, _, o = ob.decode(np.zeros((1, 2, 16), np.float32), k, v)
    return o[0, 0]


def _counts_vector(counts, n_keys):
    want = np.zeros(16)
    for t, c in counts.items():
        want[t] = c / n_keys
    return want


@pytest.mark.parametrize("chunks,want", [
    ([[1, 2, 3], [4, 5]], [2, 3, 4, 5]),          # carry 2 from a 3-token window
    ([[1, 2], [3, 4, 5]], [2, 3, 4, 5]),          # carry 1 from a 2-token window
    ([[1, 2], [3, 4]], [1, 2, 3, 4]),             # carry the whole 2-token window
    ([[1, 2], [3, 4, 5, 6, 7]], [4, 5, 6, 7]),    # T >= R: the chunk's last 4
    ([[1, 2, 3, 4, 5, 6], [7, 8]], [5, 6, 7, 8]),
    ([[1, 2]], [1, 2, 0, 0]),                     # short window: tail never written
])
def test_store_recent_window_known_answers(chunks, want):
    """Hand-derived from m12_runtime.py:482-503: recent_len = min(R, valid + T);
    T >= recent_len copies the chunk's last recent_len tokens, else carry =
    recent_len - T tokens move from recent[old - carry:old] to the front."""
    ob = O.M12Oracle(_tiny_cfg())
    for c in chunks:
        k, v = _tagged(c)
        ob.store_kv(k, v)
    assert _recent_tags(ob) == want
    assert ob.valid_len == sum(len(c) for c in chunks)


@pytest.mark.parametrize("pending,n,want", [
    ([4, 5], 1, [1, 2, 3, 4]),                    # carry 3
    ([4, 5, 6], 2, [2, 3, 4, 5]),                 # carry 2 from a 3-token window
    ([4, 5, 6, 7, 8], 5, [5, 6, 7, 8]),           # n >= R: the accepted prefix's last 4
    ([4, 5], 0, [1, 2, 3, 0]),                    # nothing accepted
])
def test_commit_known_answers(pending, n, want):
    """m12_runtime.py:777-803 on a 3-token window [1, 2, 3, _]."""
    ob = O.M12Oracle(_tiny_cfg())
    ob.store_kv(*_tagged([1, 2, 3]))
    ob.pending = _tagged(pending)
    ob.commit_verified(n)
    assert _recent_tags(ob) == want
    assert ob.valid_len == 3 + max(n, 0) and ob.pending is None


def test_short_history_decode_attends_the_shifted_stale_slots():
    """valid_len + 1 < R: decode shifts the left-aligned window left and reads
    its last valid_len + 1 slots (m12_runtime.py:1164-1172, :1290-1292), so
    the prefill tokens slide out of view and never-written slots are attended.
    R = 4, sink 2, blocks of 2: store [1, 2]; history = block 0 (protected,
    but k = max(1, 0) = 1 still selects it, the lowest id)."""
    ob = O.M12Oracle(_tiny_cfg())
    ob.store_kv(*_tagged([1, 2]))
    o = _decode_tagged(ob, 3)
    assert _recent_tags(ob) == [2, 0, 0, 3]
    assert ob.last_block_ids.tolist() == [0]
    # keys: block 0 [1, 2] | sink [1, 2] | recent[1:] = [0, 0, 3]
    assert np.allclose(o, _counts_vector({1: 2, 2: 2, 3: 1}, 7))
    o = _decode_tagged(ob, 4)
    assert _recent_tags(ob) == [0, 0, 3, 4]
    # full-length read now: recent[0:4] = [0, 0, 3, 4]
    assert np.allclose(o, _counts_vector({1: 2, 2: 2, 3: 1, 4: 1}, 8))


def test_decode_then_commit_on_a_short_window():
    """Decode (right end) then commit (left-aligned carry) while valid_len < R:
    store [1, 2] -> [1, 2, 0, 0]; decode 3 -> [2, 0, 0, 3] (valid 3); commit
    one of [4, 5]: old = 3, new = 4, carry 3 -> [2, 0, 0, 4]; decode 6 ->
    [0, 0, 4, 6].  Committing two instead: carry 2 -> [0, 0, 4, 5]."""
    for n, after_commit, after_decode in ((1, [2, 0, 0, 4], [0, 0, 4, 6]),
                                          (2, [0, 0, 4, 5], [0, 4, 5, 6])):
        ob = O.M12Oracle(_tiny_cfg())
        ob.store_kv(*_tagged([1, 2]))
        _decode_tagged(ob, 3)
        ob.pending = _tagged([4, 5])
        ob.commit_verified(n)
        assert _recent_tags(ob) == after_commit
        o = _decode_tagged(ob, 6)
        assert _recent_tags(ob) == after_decode
        counts = {1: 2, 2: 2}
        for t in after_decode:
            if t:
                counts[t] = counts.get(t, 0) + 1
        assert np.allclose(o, _counts_vector(counts, 8))


def test_store_and_commit_keep_the_last_tokens_left_aligned():
    """Closed form over random store / commit sequences with no decode: after
    every call recent[:min(R, valid_len)] is the last min(R, valid_len) tokens
    of the concatenated stream."""
    rng = np.random.default_rng(11)
    for _ in range(300):
        R = int(rng.choice([2, 3, 4, 5, 8]))
        ob = O.M12Oracle(_tiny_cfg(R=R))
        stream = []
        nxt = 1
        for op in range(int(rng.integers(1, 7))):
            if op == 0 or rng.random() < 0.5:
                T = int(rng.integers(2, 2 * R + 2))
                ids = list(range(nxt, nxt + T))
                ob.store_kv(*_tagged([t % 15 + 1 for t in ids]))
                stream += ids
            else:
                tq = int(rng.integers(1, 2 * R + 1))
                n = int(rng.integers(0, tq + 1))
                ids = list(range(nxt, nxt + tq))
                ob.pending = _tagged([t % 15 + 1 for t in ids])
                ob.commit_verified(n)
                stream += ids[:n]
                T = tq
            nxt += T
            m = min(R, ob.valid_len)
            assert ob.valid_len == len(stream)
            assert _recent_tags(ob)[:m] == [t % 15 + 1 for t in stream[len(stream) - m:]]


def test_query_summary_rounding_against_torch_mean():
    """The summary is the bf16 rounding of the exact mean; torch's bf16 mean
    (fp32 accumulation, the reference's q.mean, m12_runtime.py:53-67) agrees
    on all but rare elements whose exact mean lies next to a bf16 rounding
    boundary, and there by one bf16 ulp (measured: 1 of 12288 on three
    4096-query chunks)."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(4096, 32, 128, generator=g).to(torch.bfloat16)
    ref = q.mean(dim=0).float().numpy()
    ours = O.query_summaries(q.float().numpy(), 1)[0]
    diff = ref != ours
    assert diff.mean() <= 1e-3
    ulp = np.abs(O.bf16_round(ours * (1 + 2.0 ** -7)) - ours)
    assert (np.abs(ref - ours)[diff] <= ulp[diff] * 1.0001).all()


# ---- per-query-tile prefill selection (no reference counterpart) -----------------

def _tile_oracle(T0, seed, **kw):
    cfg = O.OracleConfig(block_size=4, r=1, recent_tokens=8, sink_tokens=4, num_heads=4, num_kv_heads=2,
                         head_dim=8, scale=0.35, **kw)
    ob = O.M12Oracle(cfg)
    rng = np.random.default_rng(seed)
    k = _rand_bf16(rng, (T0, 2, 8), 0.5)
    v = _rand_bf16(rng, (T0, 2, 8), 0.5)
    ob.store_kv(k, v)
    return ob, k, v, rng


def test_tiled_prefill_with_one_tile_is_the_chunk_routing():
    """A chunk no longer than the tile is one tile: same ids, same output as
    prefill_chunk (one query summary, m12_runtime.py:550-556)."""
    for seed in range(5):
        a, _, _, rng = _tile_oracle(64, seed, top_k_blocks=3)
        b, _, _, _ = _tile_oracle(64, seed, top_k_blocks=3)
        q = _rand_bf16(rng, (12, 4, 8))
        kn, vn = _rand_bf16(rng, (12, 2, 8), 0.5), _rand_bf16(rng, (12, 2, 8), 0.5)
        ids_t, o_t = a.prefill_chunk_tiled(q, kn, vn, tile=16)
        ids_c, o_c = b.prefill_chunk(q, kn, vn)
        assert ids_t.shape[0] == 1 and ids_t[0].tolist() == ids_c.tolist()
        assert np.array_equal(o_t, o_c)
        assert a.valid_len == b.valid_len and np.array_equal(a.recent_k, b.recent_k)


def test_tiled_prefill_selecting_everything_is_full_causal_attention():
    """With a budget above every selectable block each tile attends the whole
    history exactly once, so every query's output equals plain causal
    attention over [history | chunk] (the coverage identity of
    test_m14_prefill_layout.py:12-44)."""
    ob, k0, v0, rng = _tile_oracle(64, 3, top_k_blocks=64)
    q = _rand_bf16(rng, (40, 4, 8))
    kn, vn = _rand_bf16(rng, (40, 2, 8), 0.5), _rand_bf16(rng, (40, 2, 8), 0.5)
    ids, o = ob.prefill_chunk_tiled(q, kn, vn, tile=8)
    assert ids.shape == (5, 13)        # 16 blocks, protected {0} and the recent blocks {14, 15}
    kk, vv = np.concatenate([k0, kn]), np.concatenate([v0, vn])
    ref = O.attention_fp64(q, kk, vv, 0.35, O.causal_mask(40, 104, 64))
    assert np.allclose(o, ref, rtol=1e-12, atol=1e-12)


def test_tiled_prefill_routes_each_tile_to_its_own_blocks():
    """Two tiles whose queries point at different planted blocks select
    different blocks (budget 1): tile 0 -> block 5, tile 1 -> block 9; a
    shared selection would pick one block for both."""
    ob, _, _, rng = _tile_oracle(64, 4, top_k_blocks=1)
    da = np.zeros((4, 8), np.float32); da[:, 0] = 1.0
    db = np.zeros((4, 8), np.float32); db[:, 1] = 1.0
    reps = np.zeros_like(ob.reps)
    reps[:, 5, 0, 0] = 1.0
    reps[:, 9, 0, 1] = 1.0
    ob.reps = reps
    q = np.concatenate([np.repeat(da[None], 8, 0), np.repeat(db[None], 8, 0)]).astype(np.float32)
    kn, vn = _rand_bf16(rng, (16, 2, 8), 0.5), _rand_bf16(rng, (16, 2, 8), 0.5)
    ids, _ = ob.prefill_chunk_tiled(q, kn, vn, tile=8)
    assert ids.tolist() == [[5], [9]]
