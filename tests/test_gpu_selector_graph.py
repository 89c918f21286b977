"""The selector graph (use_graph / cfg.selector_cuda_graph): the score + top-k
launches captured in a HIP graph and replayed, with the reference's cache
lifecycle (nanovllm/sparse/m12_runtime.py:294-299, :901-957).

Restates the reference's tests/test_m19_selector_graph.py:14-150 at this
build's kernel shape (head_dim 128, 64-token blocks; the reference's toy
config uses head_dim 4 and 2-token blocks): replayed ids equal the eager
selection's, one capture serves a (history length, budget, protected set,
query shape, representatives) key, any change captures anew, reset drops
the graph and its counters, and rebuilding representatives invalidates it.
Every replay is checked against an eager selection run between replays.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 2, 1, 128


def _runtime(*, nblocks=8, dynamic_top_k=False, **kw):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    cfg = M12Config(block_size=64, r=2, recent_tokens=64, sink_tokens=64, top_k_blocks=6,
                    max_model_len=64 * 32, num_heads=HQ, num_kv_heads=HKV, head_dim=D,
                    dtype=torch.bfloat16, dynamic_top_k=dynamic_top_k, selector_cuda_graph=True, **kw)
    rt = M12LayerRuntime(0, cfg, device="cuda")
    rt.nblocks_filled = nblocks
    rt.reps_gpu[:, :nblocks].copy_(torch.randn(HKV, nblocks, cfg.r, D, device="cuda").to(torch.bfloat16))
    return rt


def _ids(rt, query, *, graph, dynamic=False, budget=None):
    return rt._gpu_select(query, use_graph=graph, dynamic=dynamic, budget=budget)[0]


def test_graph_matches_eager_for_changing_queries_and_dynamic_topk():
    torch.manual_seed(1901)
    rt = _runtime(dynamic_top_k=True)
    for _ in range(4):
        query = torch.randn(3, HQ, D, device="cuda", dtype=torch.bfloat16)
        eager = _ids(rt, query, graph=False, dynamic=True)
        graph = _ids(rt, query, graph=True, dynamic=True)
        assert torch.equal(graph, eager)
    assert rt.selector_graph_builds == 1
    assert rt.selector_graph_setup_ms > 0.0


@pytest.mark.parametrize("budget", [1, 3, 6])
def test_graph_matches_eager_for_small_budgets_and_protected_ids(budget):
    torch.manual_seed(1900 + budget)
    rt = _runtime()
    rt.protected_blocks = {0, 3, 100}   # ids beyond the history are ignored
    query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
    eager = _ids(rt, query, graph=False, budget=budget)
    graph = _ids(rt, query, graph=True, budget=budget)
    assert torch.equal(graph, eager)
    assert not ({0, 3} & set(graph.tolist()))
    assert graph.numel() == budget


def test_graph_ties_follow_eager_exact_ids():
    rt = _runtime()
    rt.reps_gpu[:, :rt.nblocks_filled].zero_()
    query = torch.zeros(HQ, D, device="cuda", dtype=torch.bfloat16)
    eager = _ids(rt, query, graph=False, budget=4)
    graph = _ids(rt, query, graph=True, budget=4)
    assert torch.equal(graph, eager)
    assert graph.tolist() == [0, 1, 2, 3]   # all scores tie: lower ids first


def test_graph_caps_budget_to_small_history_after_protected_mask():
    torch.manual_seed(1903)
    rt = _runtime(nblocks=3)
    rt.protected_blocks = {0, 20}
    query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
    eager = _ids(rt, query, graph=False, budget=6)
    graph = _ids(rt, query, graph=True, budget=6)
    assert torch.equal(graph, eager)
    assert graph.numel() == 2
    assert 0 not in graph.tolist()


def test_graph_matches_eager_when_all_in_range_blocks_are_protected():
    torch.manual_seed(1904)
    rt = _runtime(nblocks=3)
    rt.protected_blocks = {0, 1, 2, 20}
    query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
    eager = _ids(rt, query, graph=False, budget=6)
    graph = _ids(rt, query, graph=True, budget=6)
    assert torch.equal(graph, eager)
    assert graph.numel() == 1
    assert graph.item() in {0, 1, 2}


def test_graph_reuses_capture_for_current_query_and_in_place_representatives():
    torch.manual_seed(1902)
    rt = _runtime()
    for _ in range(2):
        query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
        assert torch.equal(_ids(rt, query, graph=True), _ids(rt, query, graph=False))
    builds = rt.selector_graph_builds
    # representatives edited in place (same storage): the replay reads them
    rt.reps_gpu[:, :rt.nblocks_filled].mul_(-1)
    for _ in range(3):
        query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
        assert torch.equal(_ids(rt, query, graph=True), _ids(rt, query, graph=False))
    assert rt.selector_graph_builds == builds == 1


def test_graph_rebuilds_for_shape_protection_and_budget_changes():
    torch.manual_seed(1905)
    rt = _runtime()
    query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(_ids(rt, query, graph=True, budget=4), _ids(rt, query, graph=False, budget=4))
    assert rt.selector_graph_builds == 1

    rt.nblocks_filled -= 1
    assert torch.equal(_ids(rt, query, graph=True, budget=4), _ids(rt, query, graph=False, budget=4))
    assert rt.selector_graph_builds == 2

    rt.protected_blocks.add(2)
    assert torch.equal(_ids(rt, query, graph=True, budget=4), _ids(rt, query, graph=False, budget=4))
    assert rt.selector_graph_builds == 3

    assert torch.equal(_ids(rt, query, graph=True, budget=3), _ids(rt, query, graph=False, budget=3))
    assert rt.selector_graph_builds == 4

    # a query of another shape (two summaries) captures anew as well
    q2 = torch.randn(2, HQ, D, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(_ids(rt, q2, graph=True, budget=3), _ids(rt, q2, graph=False, budget=3))
    assert rt.selector_graph_builds == 5


def test_reset_drops_graph_and_counters_and_representative_build_invalidates():
    torch.manual_seed(1906)
    rt = _runtime()
    query = torch.randn(HQ, D, device="cuda", dtype=torch.bfloat16)
    _ids(rt, query, graph=True)
    assert rt._selector_graph is not None

    rt.reset()
    assert rt._selector_graph is None
    assert rt._selector_graph_key is None
    assert rt.selector_graph_builds == 0
    assert rt.selector_graph_setup_ms == 0.0

    rt.nblocks_filled = 4
    rt.reps_gpu[:, :4].copy_(torch.randn_like(rt.reps_gpu[:, :4]))
    assert torch.equal(_ids(rt, query, graph=True), _ids(rt, query, graph=False))
    assert rt._selector_graph is not None
    assert rt.selector_graph_builds == 1

    new_keys = torch.randn(2, 64, HKV, D, device="cuda").to(torch.bfloat16)
    rt._build_reps_gpu(new_keys, start=0, nblocks=2)
    assert rt._selector_graph is None
    assert rt._selector_graph_key is None
    assert torch.equal(_ids(rt, query, graph=True), _ids(rt, query, graph=False))
    assert rt.selector_graph_builds == 2


def test_decode_with_selector_graph_matches_eager_decode():
    """decode() with cfg.selector_cuda_graph: the same ids and bit-identical
    outputs as the eager selector, one capture over the steady decode steps,
    and a new one after another prefill chunk changes the history."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    g = torch.Generator().manual_seed(1907)
    T = 64 * 40

    def rand(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).cuda()

    k = rand(T, 8, D, scale=D ** -0.5)
    v = rand(T, 8, D, scale=D ** -0.5)
    rts = []
    for graph in (False, True):
        cfg = M12Config(max_model_len=T + 1024, top_k_blocks=8, recent_tokens=512, sink_tokens=64,
                        selector_cuda_graph=graph)
        rt = M12LayerRuntime(0, cfg, device="cuda")
        rt.prefill_first(None, k, v)
        rts.append(rt)
    eager, graphed = rts
    for step in range(6):
        q = rand(1, 32, D)
        kn = rand(1, 8, D, scale=D ** -0.5)
        vn = rand(1, 8, D, scale=D ** -0.5)
        o_e = eager.decode(q, kn, vn)
        o_g = graphed.decode(q, kn, vn)
        torch.cuda.synchronize()
        assert graphed.last_block_ids.tolist() == eager.last_block_ids.tolist(), f"step {step}"
        assert torch.equal(o_g, o_e), f"step {step}"
    assert graphed.selector_graph_builds == 1
    assert eager.selector_graph_builds == 0
    # another prefill chunk: new representatives, new history length -> a new capture
    qc = rand(128, 32, D)
    kc = rand(128, 8, D, scale=D ** -0.5)
    vc = rand(128, 8, D, scale=D ** -0.5)
    oc_e = eager.prefill_chunk(qc, kc, vc)
    oc_g = graphed.prefill_chunk(qc, kc, vc)
    assert torch.equal(oc_g, oc_e)
    q = rand(1, 32, D)
    kn = rand(1, 8, D, scale=D ** -0.5)
    vn = rand(1, 8, D, scale=D ** -0.5)
    o_e = eager.decode(q, kn, vn)
    o_g = graphed.decode(q, kn, vn)
    torch.cuda.synchronize()
    assert graphed.last_block_ids.tolist() == eager.last_block_ids.tolist()
    assert torch.equal(o_g, o_e)
    assert graphed.selector_graph_builds == 2
