"""Speculative verify for all layers at once (M12ModelRuntime.verify) against the
per-layer runtime (M12LayerRuntime.verify_tokens, itself checked against the
oracle in test_gpu_store_verify.py): the same union of per-query selections
(built on the device here, on the host there), and the same ring after
commit / rollback, checked by a following decode step.

The outputs are two approximations of the same attention: the few-query
kernel's fp32 sums are split differently (one bf16 ulp apart); the
matrix-core kernel also rounds P to bf16 against each split's running max
and the two runtimes choose different split counts, so each is within
PREFILL_TOL of the exact result and they are within twice that of each other.
"""

import pytest
import torch

from tests._util import PREFILL_TOL

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _close(a, b, rel, abs_tol):
    a, b = a.float().cpu(), b.float().cpu()
    return bool(((a - b).abs() <= rel * b.abs() + abs_tol).all() and (a - b).abs().max() <= 2e-3)


@pytest.mark.parametrize("kernel", ["mfma", "few_query"])
@pytest.mark.parametrize("lossless", [True, False])
@pytest.mark.parametrize("quant", [False, True])
def test_batched_verify_matches_per_layer(lossless, quant, kernel):
    """Through the matrix-core kernel (forced with mfma_chunk_min_tokens=1:
    the union's -1 padding is passed over) and the few-query kernel (the
    automatic choice for 6 tokens, its wide 32-row form; per-layer masks
    through allowed_layer_stride, padding skipped per wavefront)."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime, M12ModelRuntime
    L, T, tq = 3, 16384, 6
    cfg = M12Config(max_model_len=T + 64, quant_history=quant,
                    mfma_chunk_min_tokens=1 if kernel == "mfma" else None)
    # verify outputs (see the module docstring); decode is the few-query kernel
    v_tol = (2 * PREFILL_TOL["rel"], 2 * PREFILL_TOL["abs_tol"]) if kernel == "mfma" else (2.0 ** -7, 1e-6)
    model = M12ModelRuntime(L, cfg)
    layers = [M12LayerRuntime(i, cfg) for i in range(L)]
    k0 = torch.stack([_rand((T, 8, 128), 500 + i, 0.09) for i in range(L)]).cuda()
    v0 = torch.stack([_rand((T, 8, 128), 600 + i, 0.09) for i in range(L)]).cuda()
    model.prefill(k0, v0)
    for i, rt in enumerate(layers):
        rt.prefill_first(None, k0[i], v0[i])
        rt.verify_lossless = lossless
    for rnd, accept in enumerate((3, 0, 6)):
        q = torch.stack([_rand((tq, 32, 128), 700 + 10 * rnd + i) for i in range(L)]).cuda()
        k = torch.stack([_rand((tq, 8, 128), 800 + 10 * rnd + i, 0.09) for i in range(L)]).cuda()
        v = torch.stack([_rand((tq, 8, 128), 900 + 10 * rnd + i, 0.09) for i in range(L)]).cuda()
        out = model.verify(q, k, v, lossless=lossless)
        for i, rt in enumerate(layers):
            o_i = rt.verify_tokens(q[i], k[i], v[i])
            ids_i = rt.last_verify_block_ids.tolist()
            if lossless:
                n = int(model.last_union_count_dev[i])
                assert model.last_union_dev[i, :n].tolist() == ids_i
                assert (model.last_union_dev[i, n:] == -1).all()
            else:
                assert sorted(model.last_union_dev[i].tolist()) == sorted(ids_i)
            assert _close(out[i], o_i, *v_tol)
            if rnd == 1:
                rt.rollback_verified()
            else:
                rt.commit_verified(accept)
        if rnd == 1:
            model.rollback_verified()
        else:
            model.commit_verified(accept)
        assert model.valid_len == layers[0].valid_len
    q = torch.stack([_rand((1, 32, 128), 1000 + i) for i in range(L)]).cuda()
    k = torch.stack([_rand((1, 8, 128), 1100 + i, 0.09) for i in range(L)]).cuda()
    v = torch.stack([_rand((1, 8, 128), 1200 + i, 0.09) for i in range(L)]).cuda()
    out = model.decode(q, k, v)
    for i, rt in enumerate(layers):
        o_i = rt.decode(q[i], k[i], v[i])
        n = model.last_n_selected
        assert model.last_ids_dev[i, 0, :n].cpu().tolist() == rt.last_block_ids.tolist()
        assert _close(out[i], o_i, 2.0 ** -7, 1e-6)


@pytest.mark.parametrize("top_k", [32, 80])
def test_lossless_verify_one_launch_selection_matches_two_launches(top_k):
    """M12ModelRuntime.verify's per-query selection in one launch
    (nkv_select_per_query, budgets up to 64) against nkv_select +
    nkv_select_union (the runtime's path above 64, forced here for 32 through
    the class switch): the same unions and the same outputs bit for bit; at
    80 the unions also against the per-layer runtime's host union."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime, M12ModelRuntime
    L, T, tq = 4, 8192, 6
    cfg = M12Config(max_model_len=T + 64, top_k_blocks=top_k)
    model = M12ModelRuntime(L, cfg)
    k0 = torch.stack([_rand((T, 8, 128), 1500 + i, 0.09) for i in range(L)]).cuda()
    v0 = torch.stack([_rand((T, 8, 128), 1600 + i, 0.09) for i in range(L)]).cuda()
    model.prefill(k0, v0)
    q = torch.stack([_rand((tq, 32, 128), 1700 + i) for i in range(L)]).cuda()
    k = torch.stack([_rand((tq, 8, 128), 1800 + i, 0.09) for i in range(L)]).cuda()
    v = torch.stack([_rand((tq, 8, 128), 1900 + i, 0.09) for i in range(L)]).cuda()
    core_cls = type(model.core)
    outs = {}
    try:
        for fused in (True, False):
            core_cls.FUSED_SELECT_UNION = fused
            o = model.verify(q, k, v, lossless=True)
            outs[fused] = (o.cpu(), model.last_union_count_dev.cpu(), model.last_union_dev.cpu())
            model.rollback_verified()
    finally:
        core_cls.FUSED_SELECT_UNION = True
    (oa, na, ua), (ob, nb, ub) = outs[True], outs[False]
    assert torch.equal(na, nb)
    for i in range(L):
        assert torch.equal(ua[i, :na[i]], ub[i, :nb[i]])
    assert torch.equal(oa.view(torch.int16), ob.view(torch.int16))
    if top_k > 64:
        for i in range(L):
            rt = M12LayerRuntime(i, cfg)
            rt.prefill_first(None, k0[i], v0[i])
            rt.verify_lossless = True
            rt.verify_tokens(q[i], k[i], v[i])
            assert ua[i, :na[i]].tolist() == rt.last_verify_block_ids.tolist()
