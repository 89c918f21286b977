"""Store, prefill-chunk and speculative-verify paths on the GPU vs the oracle.

Covers the representative builder (m12_runtime.py:354-395), query summaries
(:53-67), chunked prefill over [selected | sink | previous recent | chunk]
with store-after-attend ordering (:528-651), verify with shared and lossless
selection plus commit / rollback (:656-807), and the recent-window carry of
multi-chunk stores (:486-503).
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import PREFILL_TOL, assert_close_bf16, to_np

pytestmark = pytest.mark.gpu


def _sync_reps(rt, ob):
    nb = rt.nblocks_filled
    assert nb == ob.nblocks_filled
    ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])


def _pair(max_len, **kw):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    cfg = M12Config(max_model_len=max_len, **kw)
    rt = M12LayerRuntime(0, cfg)
    okw = {k: v for k, v in kw.items() if k in O.OracleConfig.__dataclass_fields__}
    ob = O.M12Oracle(O.OracleConfig(**okw))
    return rt, ob


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("T,r", [(4096, 4), (1000, 4), (640, 2), (200, 8)])
def test_representatives_match_oracle(T, r):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    rt = M12LayerRuntime(0, M12Config(max_model_len=T + 64, r=r))
    k = _rand((T, 8, 128), T, 128 ** -0.5)
    rt.prefill_first(None, k.cuda(), k.cuda())
    nb = rt.nblocks_filled
    kp = torch.zeros(nb * 64, 8, 128, dtype=torch.bfloat16)
    kp[:T] = k
    sel, reps, margins = O.build_reps(to_np(kp).reshape(nb, 64, 8, 128), r)
    got = rt.reps_gpu[:, :nb].cpu()
    # compare every (block, head) except near-ties: an exact tie (margin 0,
    # e.g. zero-padded rows) is decided by the first-index rule on both sides
    near = (margins > 0) & (margins <= 1e-5)
    clear = torch.from_numpy(~near.any(axis=2))                    # [nb, 8]
    want = torch.from_numpy(reps).to(torch.bfloat16)               # [8, nb, r, D]
    same = (got == want).all(dim=-1).all(dim=-1).T                 # [nb, 8]
    assert bool(same[clear].all()), f"{int((~same & clear).sum())} clear (block, head) picks differ"
    assert clear.float().mean() > 0.95


@pytest.mark.parametrize("T,nseg", [(4096, 1), (4096, 4), (10, 4), (3, 5), (1, 1)])
def test_query_summaries_bit_exact(T, nseg):
    from nanokv_amd.sparse import prefill_query_summaries
    q = _rand((T, 32, 128), 7 * T + nseg)
    got = prefill_query_summaries(q.cuda(), nseg).cpu()
    want = O.query_summaries(to_np(q), nseg)
    assert np.array_equal(to_np(got), want)


def test_prefill_chunks_then_decode_match_oracle():
    """First chunk 2048 (dense part is the caller's), later chunks of 512 and 300."""
    rt, ob = _pair(4096)
    k0, v0 = _rand((2048, 8, 128), 1, 0.09), _rand((2048, 8, 128), 2, 0.09)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    _sync_reps(rt, ob)
    for i, T in enumerate((512, 300)):
        q = _rand((T, 32, 128), 10 + i)
        k, v = _rand((T, 8, 128), 20 + i, 0.09), _rand((T, 8, 128), 30 + i, 0.09)
        out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda())
        ids_or, o_ref = ob.prefill_chunk(to_np(q), to_np(k), to_np(v))
        _sync_reps(rt, ob)
        assert rt.last_prefill_block_ids.tolist() == ids_or.tolist()
        assert_close_bf16(to_np(out), o_ref, **PREFILL_TOL)
        assert rt.valid_len == ob.valid_len and rt.prefill_len == ob.prefill_len
        assert rt.protected_blocks == ob.protected_blocks
    for s in range(3):
        q, k, v = _rand((1, 32, 128), 40 + s), _rand((1, 8, 128), 50 + s, 0.09), _rand((1, 8, 128), 60 + s, 0.09)
        out = rt.decode(q.cuda(), k.cuda(), v.cuda())
        ids_or, _, o_ref = ob.decode(to_np(q), to_np(k), to_np(v))
        assert rt.last_block_ids.tolist() == ids_or.tolist()
        assert_close_bf16(to_np(out), o_ref)


def test_small_chunks_exercise_recent_carry():
    """Chunks shorter than the recent window: the carry path of _store_kv."""
    rt, ob = _pair(2048, recent_tokens=256, sink_tokens=64, top_k_blocks=4)
    k0, v0 = _rand((100, 8, 128), 70, 0.09), _rand((100, 8, 128), 71, 0.09)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    _sync_reps(rt, ob)
    for i, T in enumerate((90, 130, 64)):
        q = _rand((T, 32, 128), 80 + i)
        k, v = _rand((T, 8, 128), 90 + i, 0.09), _rand((T, 8, 128), 100 + i, 0.09)
        out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda())
        ids_or, o_ref = ob.prefill_chunk(to_np(q), to_np(k), to_np(v))
        _sync_reps(rt, ob)
        assert rt.last_prefill_block_ids.tolist() == ids_or.tolist()
        assert_close_bf16(to_np(out), o_ref, **PREFILL_TOL)
    for s in range(4):
        q, k, v = _rand((1, 32, 128), 110 + s), _rand((1, 8, 128), 120 + s, 0.09), _rand((1, 8, 128), 130 + s, 0.09)
        out = rt.decode(q.cuda(), k.cuda(), v.cuda())
        ids_or, _, o_ref = ob.decode(to_np(q), to_np(k), to_np(v))
        assert rt.last_block_ids.tolist() == ids_or.tolist()
        assert_close_bf16(to_np(out), o_ref)


@pytest.mark.parametrize("kernel", ["mfma", "few_query"])
@pytest.mark.parametrize("lossless", [False, True])
@pytest.mark.parametrize("quant", [False, True])
def test_verify_commit_rollback_then_decode(lossless, quant, kernel):
    """6-token verify through the few-query kernel (the automatic choice: its
    wide form takes the 24 query rows as one 32-row group) and through the
    matrix-core kernel (forced with mfma_chunk_min_tokens=1)."""
    rt, ob = _pair(16384 + 64, quant_history=quant,
                   mfma_chunk_min_tokens=1 if kernel == "mfma" else None)
    k0, v0 = _rand((16384, 8, 128), 140, 0.09), _rand((16384, 8, 128), 141, 0.09)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    _sync_reps(rt, ob)
    rt.verify_lossless = lossless
    # int8: rel 2^-6 (q x scale rounded to bf16); the matrix-core kernel feeds
    # P to bf16 MFMA (PREFILL_TOL); decode after verify is the few-query kernel
    tol = dict(rel=2.0 ** -6, abs_tol=2e-4) if quant else (PREFILL_TOL if kernel == "mfma" else {})
    dec_tol = dict(rel=2.0 ** -6, abs_tol=2e-4) if quant else {}
    for rnd, accept in enumerate((3, 0, 6)):
        tq = 6
        q = _rand((tq, 32, 128), 150 + rnd)
        k, v = _rand((tq, 8, 128), 160 + rnd, 0.09), _rand((tq, 8, 128), 170 + rnd, 0.09)
        out = rt.verify_tokens(q.cuda(), k.cuda(), v.cuda())
        ids_or, o_ref = ob.verify_tokens(to_np(q), to_np(k), to_np(v), lossless=lossless)
        assert rt.last_verify_block_ids.tolist() == ids_or.tolist()
        assert_close_bf16(to_np(out), o_ref, **tol)
        if rnd == 1:
            rt.rollback_verified()
            ob.rollback_verified()
        else:
            rt.commit_verified(accept)
            ob.commit_verified(accept)
        assert rt.valid_len == ob.valid_len
    q, k, v = _rand((1, 32, 128), 180), _rand((1, 8, 128), 181, 0.09), _rand((1, 8, 128), 182, 0.09)
    out = rt.decode(q.cuda(), k.cuda(), v.cuda())
    ids_or, _, o_ref = ob.decode(to_np(q), to_np(k), to_np(v))
    assert rt.last_block_ids.tolist() == ids_or.tolist()
    assert_close_bf16(to_np(out), o_ref, **dec_tol)


def test_reset_reuses_buffers_without_inheriting_history():
    # reference tests/test_m16_dynamic_topk.py:65-85
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    rt = M12LayerRuntime(0, M12Config(max_model_len=2048))
    kv = _rand((128, 8, 128), 190, 0.09).cuda()
    rt.prefill_first(None, kv, kv)
    buf = rt.store.hist_k.data_ptr()
    assert rt.valid_len == rt.prefill_len == 128 and rt.nblocks_filled == 2
    rt.reset()
    assert rt.store.hist_k.data_ptr() == buf
    assert rt.valid_len == rt.prefill_len == rt.nblocks_filled == 0
    assert not rt.protected_blocks
    rt.prefill_first(None, kv, kv)
    assert rt.valid_len == rt.prefill_len == 128 and rt.nblocks_filled == 2


def test_non_finite_output_check_raises():
    # m12_runtime.py:1343-1344
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    rt = M12LayerRuntime(0, M12Config(max_model_len=2048, check_finite_outputs=True))
    kv = _rand((1024, 8, 128), 191, 0.09).cuda()
    rt.prefill_first(None, kv, kv)
    q = torch.full((1, 32, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="non-finite"):
        rt.decode(q, kv[:1], kv[:1])
