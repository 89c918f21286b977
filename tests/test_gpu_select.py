"""Kernels 1+2 (block scoring + Top-K) against the oracle, through the C ABI.

Scores must be bit-identical to the oracle's fp32 sequential-fma definition,
and the selected ids identical in value and order (score desc, id asc).
Edge cases follow the reference's selector tests
(tests/test_m19_selector_graph.py:47-87, test_m21_static_mask.py:36-101,
test_m16_dynamic_topk.py:25-63): protected ids, budget caps, all-protected
histories, exact ties, dynamic budgets.
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import f32_bits, to_np

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _runtime(nblocks, *, r=4, top_k=32, max_blocks=None, **kw):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    cfg = M12Config(top_k_blocks=top_k, r=r, max_model_len=64 * (max_blocks or nblocks), **kw)
    rt = M12LayerRuntime(0, cfg)
    rt.nblocks_filled = nblocks
    return rt


def _rand_reps(nb, r, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(HKV, nb, r, D, generator=g) / D ** 0.5).to(torch.bfloat16)


def _rand_q(nq, seed):
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randn(nq, HQ, D, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("nb,r,nq,prot,budget,seed", [
    (512, 4, 1, "std", 32, 0),       # 32K decode shape
    (128, 4, 1, "std", 32, 1),       # 8K
    (2048, 4, 1, "std", 32, 2),      # 128K
    (256, 4, 6, "std", 32, 3),       # verify: 6 queries max-reduced
    (37, 4, 1, "std", 32, 4),        # ragged tile
    (1, 4, 1, "none", 32, 5),        # one block
    (300, 2, 3, {0, 3, 299, 1000}, 24, 6),
    (64, 8, 1, "none", 16, 7),
    (100, 1, 2, "std", 48, 8),
    (1024, 4, 1, "std", 200, 9),     # wavefront top-k, k > 64: LDS sort path
    (4096, 4, 1, "std", 64, 10),     # past 2048 blocks: workgroup top-k kernel
    (3000, 2, 1, "std", 300, 11),    # workgroup kernel, ragged, large k
])
def test_scores_and_ids_bit_exact(nb, r, nq, prot, budget, seed):
    rt = _runtime(nb, r=r, top_k=max(budget, 32))
    reps = _rand_reps(nb, r, seed)
    rt.reps_gpu[:, :nb].copy_(reps.cuda())
    if prot == "std":
        rt.protected_blocks = O.protected_blocks_after_store(nb, 512, 64)
    elif prot == "none":
        rt.protected_blocks = set()
    else:
        rt.protected_blocks = set(prot)
    q = _rand_q(nq, seed)
    ids, info = rt._gpu_select(q.cuda(), budget=budget)
    scores_gpu = rt._core._last_scores[0, 0].cpu().numpy()

    s_or = O.block_scores(to_np(q), to_np(reps), nb, HKV)
    ids_or, vals_or = O.topk_blocks(s_or, rt.protected_blocks, budget)
    assert np.array_equal(f32_bits(scores_gpu), f32_bits(s_or)), "scores differ from the oracle"
    assert ids.tolist() == ids_or.tolist()
    assert info["n_selected"] == info["n_candidates"] == len(ids_or)


def test_per_query_topk_matches_oracle():
    nb, tq = 256, 6
    rt = _runtime(nb)
    reps = _rand_reps(nb, 4, 11)
    rt.reps_gpu[:, :nb].copy_(reps.cuda())
    rt.protected_blocks = O.protected_blocks_after_store(nb, 512, 64)
    q = _rand_q(tq, 11)
    union, allowed = rt._gpu_select_per_query(q.cuda(), 32)
    u_or, a_or, _ = O.select_per_query(to_np(q), to_np(reps), nb, HKV, rt.protected_blocks, 32)
    assert union.tolist() == u_or.tolist()
    assert np.array_equal(allowed.cpu().numpy(), a_or)


@pytest.mark.parametrize("budget", [1, 3, 6])
def test_protected_ids_and_small_budgets(budget):
    # test_m19_selector_graph.py:47-56: protected ids (and ids beyond history) never selected
    nb = 8
    rt = _runtime(nb, top_k=6, max_blocks=32)
    rt.reps_gpu[:, :nb].copy_(_rand_reps(nb, 4, 19).cuda())
    rt.protected_blocks = {0, 3, 100}
    ids, _ = rt._gpu_select(_rand_q(1, 19)[0].cuda(), budget=budget)
    assert ids.numel() == budget
    assert not ({0, 3} & set(ids.tolist()))


def test_budget_capped_by_history_after_protection():
    # test_m19_selector_graph.py:68-76
    rt = _runtime(3, top_k=6, max_blocks=32)
    rt.reps_gpu[:, :3].copy_(_rand_reps(3, 4, 23).cuda())
    rt.protected_blocks = {0, 20}
    ids, info = rt._gpu_select(_rand_q(1, 23)[0].cuda(), budget=6)
    assert ids.numel() == 2 and 0 not in ids.tolist()
    assert info["n_candidates"] == 2


def test_all_protected_returns_one_block_lowest_id():
    # test_m19_selector_graph.py:79-87 / test_m21_static_mask.py:80-90: k collapses to 1;
    # every score is -inf, the id-ascending tie rule picks block 0.
    rt = _runtime(4, top_k=6, max_blocks=32)
    rt.reps_gpu[:, :4].copy_(_rand_reps(4, 4, 29).cuda())
    rt.protected_blocks = {0, 1, 2, 3, 20}
    ids, info = rt._gpu_select(_rand_q(1, 29)[0].cuda(), budget=6)
    assert ids.tolist() == [0]
    assert info["n_candidates"] == 1


def test_exact_ties_take_lowest_ids():
    # test_m21_static_mask.py:28-45: all-zero reps and query -> every score is 0
    nb = 8
    rt = _runtime(nb, top_k=6, max_blocks=32)
    rt.reps_gpu[:, :nb].zero_()
    rt.protected_blocks = {0, 4, 100}
    ids, info = rt._gpu_select(torch.zeros(HQ, D, dtype=torch.bfloat16, device="cuda"), budget=6)
    assert ids.tolist() == [1, 2, 3, 5, 6, 7]
    assert info["n_selected"] == 6


def test_dynamic_budget_changes_decode_only():
    # test_m16_dynamic_topk.py:25-43: one dominant block -> dynamic budget 16 of 32
    rt = _runtime(40, top_k=32, max_blocks=128, dynamic_top_k=True)
    rt.reps_gpu.zero_()
    rt.reps_gpu[0, 0, 0, 0] = 10.0
    query = torch.zeros(1, HQ, D, dtype=torch.bfloat16, device="cuda")
    query[0, 0, 0] = 1.0
    prefill_ids, _ = rt._gpu_select(query)
    decode_ids, info = rt._gpu_select(query, dynamic=True)
    assert prefill_ids.numel() == 32
    assert decode_ids.numel() == info["n_selected"] == 16
    assert torch.equal(decode_ids, prefill_ids[:16])
    assert prefill_ids.tolist() == list(range(32))


def test_fixed_decode_override_keeps_prefill_budget():
    # test_m16_dynamic_topk.py:46-63
    rt = _runtime(40, top_k=32, max_blocks=128, decode_top_k_blocks=24)
    rt.reps_gpu.zero_()
    query = torch.zeros(1, HQ, D, dtype=torch.bfloat16, device="cuda")
    prefill_ids, _ = rt._gpu_select(query)
    decode_ids, info = rt._gpu_select(query, budget=rt.cfg.decode_top_k_blocks)
    assert prefill_ids.numel() == 32
    assert decode_ids.numel() == info["n_selected"] == 24


def test_gather_sort_orders_ids_ascending_on_device():
    from nanokv_amd import _lib
    nb = 512
    rt = _runtime(nb)
    reps = _rand_reps(nb, 4, 31)
    rt.reps_gpu[:, :nb].copy_(reps.cuda())
    rt.protected_blocks = O.protected_blocks_after_store(nb, 512, 64)
    q = _rand_q(1, 31)
    ids, _, k = rt._select_dev(q.cuda(), 32, _lib.NKV_ORDER_ID_ASC)
    got = ids[0, 0, :k].cpu().tolist()
    s_or = O.block_scores(to_np(q), to_np(reps), nb, HKV)
    ids_or, _ = O.topk_blocks(s_or, rt.protected_blocks, 32)
    assert got == sorted(ids_or.tolist())


def test_select_rejects_empty_history():
    rt = _runtime(0, max_blocks=8)
    with pytest.raises(ValueError, match="history block"):
        rt._gpu_select(_rand_q(1, 0)[0].cuda())


@pytest.mark.parametrize("L,tq,k,k_eff,hi,seed", [
    (3, 6, 32, 32, 120, 0),     # verify shape, heavy overlap between queries
    (2, 6, 32, 29, 4000, 1),    # k_eff < k, few duplicates
    (1, 1, 8, 8, 100, 2),       # one query: the union is its sorted ids
    (2, 16, 256, 256, 9000, 3), # the largest supported union (4096 ids)
    (2, 4, 64, 64, 12288, 4),   # ids up to the largest block id a selection returns
])
def test_select_union_matches_unique_and_searchsorted(L, tq, k, k_eff, hi, seed):
    """nkv_select_union against the reference's host ops (m12_runtime.py:1057-1087):
    torch.unique of the per-query ids, searchsorted, scatter into the mask."""
    from nanokv_amd.store import SparseKVStore
    rng = np.random.default_rng(seed)
    ids = np.full((L, tq, k), -7, dtype=np.int32)          # entries past k_eff must be ignored
    for l in range(L):
        for t in range(tq):
            ids[l, t, :k_eff] = rng.choice(hi, size=k_eff, replace=False)
    umax = tq * k_eff + 5
    st = SparseKVStore(1, num_heads=32, num_kv_heads=8, head_dim=128, block_size=64, r=4,
                       cap_blocks=8, sink_tokens=64, recent_tokens=512, kv_format="bf16")
    d_ids = torch.from_numpy(ids).cuda()
    union = torch.full((L, umax), 123, dtype=torch.int32, device="cuda")
    count = torch.zeros(L, dtype=torch.int32, device="cuda")
    allowed = torch.full((L, tq, umax), 9, dtype=torch.uint8, device="cuda")
    st.select_union(d_ids, k_eff, umax, union, count, allowed)
    union, count, allowed = union.cpu().numpy(), count.cpu().numpy(), allowed.cpu().numpy()
    for l in range(L):
        u = np.unique(ids[l, :, :k_eff])
        assert count[l] == u.size
        assert np.array_equal(union[l, :u.size], u)
        assert (union[l, u.size:] == -1).all()
        want = np.zeros((tq, umax), dtype=np.uint8)
        for t in range(tq):
            want[t, np.searchsorted(u, ids[l, t, :k_eff])] = 1
        assert np.array_equal(allowed[l], want)


@pytest.mark.parametrize("L,nq,nb,k,prot,seed", [
    (36, 6, 256, 32, (), 0),                 # the 36-layer 16K verify round: 6 queries, J = 8
    (3, 16, 700, 64, (0, 5, 699), 1),        # 16 queries, k = 64, 11 wavefront rows each: J = 16
    (2, 1, 2048, 17, (3, 3, 4000, -1), 2),   # one query, J = 32; repeated / outside protected ids
    (2, 3, 40, 64, (1,), 3),                 # k above the selectable blocks (k_eff 39)
    (2, 5, 100, 32, tuple(range(90)), 4),    # 10 selectable blocks: k_eff 10
    (1, 9, 513, 1, (), 5),                   # k = 1, a ragged 9th tile
])
def test_select_per_query_matches_select_then_union(L, nq, nb, k, prot, seed):
    """nkv_select_per_query (per-query Top-K and union in one launch) gives the
    bytes of nkv_select(per_query) followed by nkv_select_union: scores, ids
    (rows past k_eff untouched), values, union, counts and mask identical, the
    score keys left zeroed; a sampled layer against the oracle's
    select_per_query (m12_runtime.py:1057-1087)."""
    from nanokv_amd import _lib
    from nanokv_amd.store import SparseKVStore
    st = SparseKVStore(L, num_heads=HQ, num_kv_heads=HKV, head_dim=D, block_size=64, r=4, cap_blocks=nb,
                       sink_tokens=64, recent_tokens=512, kv_format="bf16")
    g = torch.Generator().manual_seed(seed)
    reps = (torch.randn(L, HKV, nb, 4, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    st.reps[:, :, :nb].copy_(reps.cuda())
    q = torch.randn(L, nq, HQ, D, generator=g).to(torch.bfloat16)
    prot_dev = torch.tensor(list(prot) or [0], dtype=torch.int32, device="cuda")
    k_eff = min(k, max(1, nb - len({p for p in prot if 0 <= p < nb})))
    umax = nq * min(k, nb)
    dev = "cuda"

    def outs():
        return (torch.zeros(L * nq * nb, dtype=torch.int32, device=dev),
                torch.full((L * nq * nb,), -3.0, dtype=torch.float32, device=dev),
                torch.full((L, nq, k), -5, dtype=torch.int32, device=dev),
                torch.full((L, nq, k), -7.0, dtype=torch.float32, device=dev),
                torch.full((L, umax), 123, dtype=torch.int32, device=dev),
                torch.zeros(L, dtype=torch.int32, device=dev),
                torch.full((L, nq, umax), 9, dtype=torch.uint8, device=dev))

    a = outs()
    st.select(0, q.cuda(), nb, prot_dev, len(prot), k, _lib.NKV_ORDER_SCORE_DESC, True, a[0], a[1], a[2], a[3])
    st.select_union(a[2], k_eff, umax, a[4], a[5], a[6])
    b = outs()
    st.select_per_query(0, q.cuda(), nb, prot_dev, len(prot), k, b[0], b[1], b[2], b[3], umax, b[4], b[5], b[6])
    torch.cuda.synchronize()
    assert not b[0].any(), "score keys not left zeroed"
    for name, x, y in zip(("scores", "ids", "vals", "union", "count", "allowed"), a[1:], b[1:]):
        assert torch.equal(x.cpu().view(torch.int32) if x.dtype == torch.float32 else x.cpu(),
                           y.cpu().view(torch.int32) if y.dtype == torch.float32 else y.cpu()), name
    lyr = L - 1
    u_or, a_or, tops = O.select_per_query(to_np(q[lyr]), to_np(reps[lyr]), nb, HKV, set(prot), k)
    cnt = int(b[5][lyr])
    assert tops.shape[1] == k_eff
    assert b[2][lyr, :, :k_eff].cpu().numpy().tolist() == tops.tolist()
    assert cnt == u_or.size and b[4][lyr, :cnt].cpu().tolist() == u_or.tolist()
    assert (b[4][lyr, cnt:].cpu() == -1).all()
    assert np.array_equal(b[6][lyr, :, :cnt].cpu().numpy().astype(bool), a_or)
    assert not b[6][lyr, :, cnt:].cpu().any()


def test_select_per_query_rejects_shapes_outside_its_limits():
    from nanokv_amd.store import SparseKVStore
    st = SparseKVStore(1, num_heads=HQ, num_kv_heads=HKV, head_dim=D, block_size=64, r=4, cap_blocks=4096,
                       sink_tokens=64, recent_tokens=512, kv_format="bf16")
    prot = torch.zeros(1, dtype=torch.int32, device="cuda")
    for nq, nb, k, match in ((17, 256, 32, "nq must be"), (6, 256, 65, "k must be"), (2, 2049, 32, "nblocks 2049 exceeds")):
        q = torch.zeros(1, nq, HQ, D, dtype=torch.bfloat16, device="cuda")
        keys = torch.zeros(nq * nb, dtype=torch.int32, device="cuda")
        f = torch.empty(nq * nb, dtype=torch.float32, device="cuda")
        ids = torch.empty(1, nq, k, dtype=torch.int32, device="cuda")
        vals = torch.empty(1, nq, k, dtype=torch.float32, device="cuda")
        umax = nq * min(k, nb)
        u = torch.empty(1, umax, dtype=torch.int32, device="cuda")
        c = torch.empty(1, dtype=torch.int32, device="cuda")
        al = torch.empty(1, nq, umax, dtype=torch.uint8, device="cuda")
        with pytest.raises(ValueError, match=match):
            st.select_per_query(0, q, nb, prot, 0, k, keys, f, ids, vals, umax, u, c, al)
        with pytest.raises(ValueError, match="umax"):
            st.select_per_query(0, q[:, :1], 8, prot, 0, 4, keys, f, ids, vals, 3, u, c, al)


def _pattern_reps(pattern, nb, r, seed):
    """Representatives whose scores tie a lot: 'zero_half' (every other block
    all-zero: score 0), 'levels' (reps = +-1/16 patterns shared by groups of
    blocks: a handful of distinct scores), 'equal' (all zero)."""
    g = torch.Generator().manual_seed(seed)
    reps = torch.randn(HKV, nb, r, D, generator=g) / D ** 0.5
    if pattern == "zero_half":
        reps[:, ::2] = 0.0
    elif pattern == "levels":
        base = torch.sign(torch.randn(HKV, 5, r, D, generator=g)) / 16
        reps = base[:, torch.randint(0, 5, (nb,), generator=g)]
    elif pattern == "equal":
        reps.zero_()
    return reps.to(torch.bfloat16)


@pytest.mark.parametrize("pattern", ["random", "zero_half", "levels", "equal"])
@pytest.mark.parametrize("nb,budget", [(40, 32), (512, 32), (512, 64), (2048, 1), (700, 48)])
def test_topk_short_candidate_path_and_full_search_give_the_same_ids(pattern, nb, budget):
    """The wave top-k ranks a short candidate list when at most 64 keys reach
    the k-th largest lane maximum and searches all keys otherwise (ties,
    equal scores); either way the ids equal the oracle's (score desc, id asc)."""
    rt = _runtime(nb, top_k=max(budget, 32))
    reps = _pattern_reps(pattern, nb, 4, nb + budget)
    rt.reps_gpu[:, :nb].copy_(reps.cuda())
    rt.protected_blocks = O.protected_blocks_after_store(nb, 512, 64)
    q = _rand_q(1, nb)
    ids, _ = rt._gpu_select(q.cuda(), budget=budget)
    s_or = O.block_scores(to_np(q), to_np(reps), nb, HKV)
    ids_or, _ = O.topk_blocks(s_or, rt.protected_blocks, budget)
    assert ids.tolist() == ids_or.tolist()
