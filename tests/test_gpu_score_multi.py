"""The multi-query scorer (nkv_select with nq >= 2 queries and nq * G >= 8
query rows: verify draft tokens, prefill tile summaries) against the oracle.

Each workgroup copies 32 blocks of representative rows into LDS (two rows
a lane) and splits the nq * G query rows of its KV head over four waves, so
one query's rows can be scored by two waves and combined by the atomicMax on
the order-preserving key.  Scores must be bit-identical to the oracle's sequential-fma dots
(m12_runtime.py:999-1003 and :1068-1072, the shared and per-query maxima),
and the per-query / shared Top-K ids identical, over GQA ratios 1-16, r 1-8,
ragged tiles, several layers and query-row counts that leave a short last
group.  In both scorer forms a NaN representative makes its block's score
NaN, as numpy's max over the dots does (NaN sorts above +inf).
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import to_np

pytestmark = pytest.mark.gpu

HKV, D = 8, 128


def _store(L, G, r, cap):
    from nanokv_amd.store import SparseKVStore
    return SparseKVStore(L, num_heads=HKV * G, num_kv_heads=HKV, head_dim=D, block_size=64, r=r,
                         cap_blocks=cap, sink_tokens=64, recent_tokens=512)


def _run(st, q, nb, k, per_query):
    from nanokv_amd import _lib
    L, nq = q.shape[0], q.shape[1]
    nqo = nq if per_query else 1
    dev = q.device
    keys = torch.zeros(L * nqo * nb, dtype=torch.int32, device=dev)
    scores = torch.full((L, nqo, nb), 7.0, dtype=torch.float32, device=dev)
    ids = torch.full((L, nqo, k), -5, dtype=torch.int32, device=dev)
    vals = torch.zeros((L, nqo, k), dtype=torch.float32, device=dev)
    prot = torch.zeros(1, dtype=torch.int32, device=dev)
    st.select(0, q, nb, prot, 0, k, _lib.NKV_ORDER_SCORE_DESC, per_query, keys, scores, ids, vals)
    torch.cuda.synchronize()
    assert int(keys.count_nonzero()) == 0, "the key workspace must be left zeroed"
    return scores.cpu().numpy(), ids.cpu().numpy()


@pytest.mark.parametrize("G,r,nq,nb,per_query,L,seed", [
    (4, 4, 6, 256, True, 3, 0),     # verify: 6 draft tokens (24 rows, 6 per wave)
    (4, 4, 64, 520, True, 2, 1),    # prefill tile summaries: 64 tiles (256 rows, groups of 4)
    (4, 4, 5, 100, True, 2, 2),     # 5 rows per wave (one group of 6, one repeated row)
    (4, 4, 7, 37, True, 1, 3),      # 7 rows per wave (groups of 4 and 3), ragged tile
    (1, 8, 8, 70, True, 1, 4),      # G = 1: one row per query, 2 queries per wave
    (8, 1, 2, 129, True, 2, 5),     # G = 8: each query's 8 heads split over 2 waves
    (2, 2, 6, 300, True, 1, 6),     # 12 rows: 3 per wave, queries straddle waves
    (16, 4, 3, 64, False, 2, 7),    # shared maximum over 3 queries, G = 16
    (4, 4, 6, 256, False, 2, 8),    # shared verify selection
    (4, 2, 2, 1, True, 1, 9),       # one block
])
def test_multi_query_scores_and_ids_bit_exact(G, r, nq, nb, per_query, L, seed):
    torch.manual_seed(4100 + seed)
    st = _store(L, G, r, max(nb, 8))
    reps = (torch.randn(L, HKV, nb, r, D) / D ** 0.5).to(torch.bfloat16)
    st.reps[:, :, :nb].copy_(reps.cuda())
    q = torch.randn(L, nq, HKV * G, D).to(torch.bfloat16)
    k = min(8, nb)
    scores, ids = _run(st, q.cuda(), nb, k, per_query)
    for l in range(L):
        if per_query:
            s_or = O.block_scores_per_query(to_np(q[l]), to_np(reps[l]), nb, HKV)     # [nq, nb]
        else:
            s_or = O.block_scores(to_np(q[l]), to_np(reps[l]), nb, HKV)[None]          # [1, nb]
        assert np.array_equal(O.orderable_key(scores[l]), O.orderable_key(s_or)), f"layer {l}: scores differ"
        for t in range(s_or.shape[0]):
            ids_or, _ = O.topk_blocks(s_or[t], set(), k)
            assert ids[l, t].tolist() == ids_or.tolist(), f"layer {l} row {t}: ids differ"


@pytest.mark.parametrize("nq,per_query", [(6, True), (6, False), (1, False), (1, True), (2, False)])
def test_nan_representative_makes_the_block_score_nan(nq, per_query):
    """Both scorer forms (one query: score_kernel; several: score_multi_kernel)."""
    torch.manual_seed(4200 + nq)
    G, r, nb = 4, 4, 48
    st = _store(1, G, r, nb)
    reps = (torch.randn(1, HKV, nb, r, D) / D ** 0.5).to(torch.bfloat16)
    reps[0, 3, 17, 2, 40] = float("nan")     # one element of one representative of block 17
    reps[0, 5, 30, 0, :] = float("inf")      # inf products of both signs: NaN dots for block 30
    st.reps[:, :, :nb].copy_(reps.cuda())
    q = torch.randn(1, nq, HKV * G, D).to(torch.bfloat16)
    scores, ids = _run(st, q.cuda(), nb, 4, per_query)
    if per_query:
        s_or = O.block_scores_per_query(to_np(q[0]), to_np(reps[0]), nb, HKV)
    else:
        s_or = O.block_scores(to_np(q[0]), to_np(reps[0]), nb, HKV)[None]
    assert np.isnan(s_or[:, 17]).all() and np.isnan(s_or[:, 30]).all()
    assert np.array_equal(O.orderable_key(scores[0]), O.orderable_key(s_or))
    for t in range(s_or.shape[0]):
        ids_or, _ = O.topk_blocks(s_or[t], set(), 4)
        assert ids[0, t].tolist() == ids_or.tolist()
        assert ids[0, t, :2].tolist() == [17, 30]    # NaN above every finite score, lower id first
