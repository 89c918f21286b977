"""Decode layer-step (select + in-place gather + segmented attention) vs the oracle.

A runtime is prefilled, then stepped; after every step the selected ids must
equal the oracle's (value and order) and the bf16 output must match the fp64
oracle to about one bf16 ulp (and always within the 2e-3 max-abs bar).  The
oracle replays the reference's semantics including the recent-window shift
(m12_runtime.py:1164-1172), the frozen history / protected set, and the
reference's int8 dequantisation into bf16 before attention
(m12_runtime.py:1262-1267).

The oracle is given the representatives the GPU built (the representative
builder has its own test), so these tests isolate the decode path.
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import assert_close_bf16, to_np

pytestmark = pytest.mark.gpu


def _make(T, steps, seed, *, quant=False, layout="channel_block", recent=512, sink=64,
          top_k=32, planted=3, gather_sort=False, decode_budget=None, **policy):
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    cfg = M12Config(max_model_len=T + 64, quant_history=quant, quant_scale_layout=layout,
                    recent_tokens=recent, sink_tokens=sink, top_k_blocks=top_k,
                    gather_sort=gather_sort, decode_top_k_blocks=decode_budget, **policy)
    rt = M12LayerRuntime(0, cfg)
    k, v, q, planted_ids = workload.history(T, seed, num_planted=planted, recent_tokens=recent)
    rt.prefill_first(None, k.cuda(), v.cuda())
    ocfg = O.OracleConfig(recent_tokens=recent, sink_tokens=sink, top_k_blocks=top_k,
                          quant_history=quant and layout == "channel_block",
                          decode_top_k_blocks=decode_budget, **policy)
    ob = O.M12Oracle(ocfg)
    ob.store_kv(to_np(k), to_np(v), with_reps=False)
    nb = rt.nblocks_filled
    assert nb == ob.nblocks_filled
    ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])
    qs, ks, vs = workload.decode_inputs(steps, seed)
    return rt, ob, q, planted_ids, (qs, ks, vs)


def _dequant_token_layout(ob, rt):
    """Give the oracle the per-token fp16-scale history the GPU stored."""
    st = rt.store
    nb = rt.nblocks_filled
    kq = st.hist_k[0, :, :nb].cpu().numpy().astype(np.float32)          # [H, nb, 64, D]
    vq = st.hist_v[0, :, :nb].cpu().numpy().astype(np.float32)
    ks = st.k_tscale[0, :, :nb * 64].cpu().float().numpy().reshape(8, nb, 64, 1)
    vsc = st.v_tscale[0, :, :nb * 64].cpu().float().numpy().reshape(8, nb, 64, 1)
    ob.hist_k[:nb] = O.bf16_round(kq * ks).transpose(1, 2, 0, 3)
    ob.hist_v[:nb] = O.bf16_round(vq * vsc).transpose(1, 2, 0, 3)


def _run_steps(rt, ob, inputs, steps, *, rel=2.0 ** -7, abs_tol=2e-5, first_q=None):
    qs, ks, vs = inputs
    worst = 0.0
    for s in range(steps):
        q = qs[s, 0] if (s > 0 or first_q is None) else first_q.unsqueeze(0)
        out = rt.decode(q.cuda(), ks[s, 0].cuda(), vs[s, 0].cuda())
        ids_or, _, o_ref = ob.decode(to_np(q), to_np(ks[s, 0]), to_np(vs[s, 0]))
        got = rt.last_block_ids.tolist()
        if rt.cfg.gather_sort:
            ids_or = np.sort(ids_or)
        assert got == ids_or.tolist(), f"step {s}: ids differ"
        worst = max(worst, assert_close_bf16(to_np(out), o_ref, rel=rel, abs_tol=abs_tol))
        assert rt.valid_len == ob.valid_len
    return worst


def test_decode_8k_planted_blocks_selected():
    # 8K history, 128 blocks, protected {0, 120..127}; the planted blocks win.
    rt, ob, q, planted, inputs = _make(8192, 4, seed=1234)
    assert rt.protected_blocks == ob.protected_blocks == ({0} | set(range(120, 128)))
    out = rt.decode(q.unsqueeze(0).cuda(), inputs[1][0, 0].cuda(), inputs[2][0, 0].cuda())
    ids_or, _, o_ref = ob.decode(to_np(q.unsqueeze(0)), to_np(inputs[1][0, 0]), to_np(inputs[2][0, 0]))
    ids = rt.last_block_ids.tolist()
    assert ids == ids_or.tolist()
    assert set(planted) <= set(ids[:3])
    assert_close_bf16(to_np(out), o_ref)


@pytest.mark.parametrize("T,steps,seed", [
    (32768, 6, 7),     # the 32K headline shape
    (1000, 5, 8),      # partial last block, history shorter than sink+recent
    (4096, 3, 9),
    (131072, 2, 10),   # 2048 blocks
])
def test_decode_bf16_matches_oracle(T, steps, seed):
    rt, ob, _, _, inputs = _make(T, steps, seed)
    _run_steps(rt, ob, inputs, steps)


def test_decode_short_history_and_small_windows():
    # history shorter than the recent window: the reference's left-aligned
    # buffer semantics (stale zero slots) are reproduced exactly.
    rt, ob, _, _, inputs = _make(300, 6, 21, recent=256, sink=32, top_k=4, planted=0)
    _run_steps(rt, ob, inputs, 6)


def test_decode_gather_sort_and_budget():
    rt, ob, _, _, inputs = _make(16384, 3, 22, gather_sort=True, decode_budget=24)
    _run_steps(rt, ob, inputs, 3)


@pytest.mark.parametrize("a,cap,union", [(0.97, 48, False), (0.97, 12, True), (0.5, 20, False)])
def test_decode_relative_threshold_policy(a, cap, union):
    """decode_relative_a (m12_runtime.py:1015-1031): the kept blocks and the
    attention over them match the oracle at every step; the count varies."""
    rt, ob, _, _, inputs = _make(16384, 6, 24, decode_relative_a=a, decode_relative_max_blocks=cap,
                                 decode_relative_union=union)
    counts = []
    qs, ks, vs = inputs
    for s in range(6):
        out = rt.decode(qs[s, 0].cuda(), ks[s, 0].cuda(), vs[s, 0].cuda())
        ids_or, _, o_ref = ob.decode(to_np(qs[s, 0]), to_np(ks[s, 0]), to_np(vs[s, 0]))
        assert rt.last_block_ids.tolist() == ids_or.tolist(), f"step {s}: ids differ"
        assert_close_bf16(to_np(out), o_ref)
        counts.append(len(ids_or))
    print(f"[relative a={a} cap={cap} union={union}] kept blocks per step: {counts}", flush=True)
    assert max(counts) <= max(cap, 32 if union else 0)


@pytest.mark.parametrize("window", [2, 4])
def test_decode_query_window_policy(window):
    """decode_query_window (m12_runtime.py:1176-1189): routing on the mean of
    the last W decode queries, attention on the current one."""
    rt, ob, _, _, inputs = _make(8192, 7, 25, decode_query_window=window)
    _run_steps(rt, ob, inputs, 7)


def test_decode_many_steps_ring_wraps():
    # 520 steps: the 512-slot ring wraps; prefill tokens scroll out of the window.
    rt, ob, _, _, inputs = _make(2048, 520, 23, top_k=8, planted=0)
    qs, ks, vs = inputs
    for s in range(520):
        out = rt.decode(qs[s, 0].cuda(), ks[s, 0].cuda(), vs[s, 0].cuda())
        ids_or, _, o_ref = ob.decode(to_np(qs[s, 0]), to_np(ks[s, 0]), to_np(vs[s, 0]))
        if s % 37 == 0 or s >= 510:
            assert rt.last_block_ids.tolist() == ids_or.tolist()
            assert_close_bf16(to_np(out), o_ref)


def test_decode_int8_channel_block_matches_oracle():
    rt, ob, _, _, inputs = _make(32768, 4, 31, quant=True)
    # the GPU-stored int8 history and scales equal the oracle's bit for bit
    nb = rt.nblocks_filled
    st = rt.store
    assert np.array_equal(st.k_scale[0].cpu().numpy(), ob.k_scale)
    assert np.array_equal(st.v_scale[0, :, :nb].cpu().numpy(), ob.v_scale[:nb].T)
    assert np.array_equal(st.hist_k[0, :, :nb].cpu().numpy().transpose(1, 2, 0, 3), ob.hist_kq[:nb])
    assert np.array_equal(st.hist_v[0, :, :nb].cpu().numpy().transpose(1, 2, 0, 3), ob.hist_vq[:nb])
    worst = _run_steps(rt, ob, inputs, 4, rel=2.0 ** -6, abs_tol=2e-4)
    print(f"int8 channel/block decode max |err| = {worst:.3e}")


def test_decode_int8_token_scales_matches_oracle():
    rt, ob, _, _, inputs = _make(8192, 3, 41, quant=True, layout="token")
    nb = rt.nblocks_filled
    k, v = ob.hist_k[:nb].copy(), ob.hist_v[:nb].copy()
    # per-token fp16 scale layout: scales and int8 codes bit-exact vs the closed form
    ks_or = O.token_scale_fp16(k.transpose(2, 0, 1, 3))            # [H, nb, 64]
    vs_or = O.token_scale_fp16(v.transpose(2, 0, 1, 3))
    st = rt.store
    assert np.array_equal(st.k_tscale[0, :, :nb * 64].cpu().numpy().reshape(8, nb, 64), ks_or)
    assert np.array_equal(st.v_tscale[0, :, :nb * 64].cpu().numpy().reshape(8, nb, 64), vs_or)
    kq_or = O.quantize(k.transpose(2, 0, 1, 3), ks_or.astype(np.float32)[..., None])
    assert np.array_equal(st.hist_k[0, :, :nb].cpu().numpy(), kq_or)
    _dequant_token_layout(ob, rt)
    worst = _run_steps(rt, ob, inputs, 3, rel=2.0 ** -6, abs_tol=2e-4)
    print(f"int8 per-token decode max |err| = {worst:.3e}")


def test_model_runtime_batches_layers_like_per_layer_runtimes():
    """M12ModelRuntime (one launch per stage for all layers) == per-layer runtimes.

    Selection is bit-identical.  The attention is split into workgroup ranges
    over all (layer, KV head) pairs of a launch, so the fp32 summation order
    (not the math) depends on how many layers share the launch: outputs agree
    to one bf16 ulp.
    """
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime, M12ModelRuntime
    L, T, steps = 3, 4096, 3
    cfg = M12Config(max_model_len=T + 64)
    model = M12ModelRuntime(L, cfg)
    layers = [M12LayerRuntime(i, cfg) for i in range(L)]
    hist = [workload.history(T, 100 + i) for i in range(L)]
    k = torch.stack([h[0] for h in hist]).cuda()
    v = torch.stack([h[1] for h in hist]).cuda()
    model.prefill(k, v)
    for i, rt in enumerate(layers):
        rt.prefill_first(None, k[i], v[i])
    qs, ks, vs = workload.decode_inputs(steps, 5, layers=L)
    for s in range(steps):
        out = model.decode(qs[s].cuda(), ks[s].cuda(), vs[s].cuda())
        for i, rt in enumerate(layers):
            o_i = rt.decode(qs[s, i].cuda(), ks[s, i].cuda(), vs[s, i].cuda())
            assert torch.equal(model.last_ids_dev[i, 0, :model.last_n_selected].cpu(),
                               rt.last_block_ids.to(torch.int32))
            a, b = out[i].float().cpu(), o_i.float().cpu()
            assert ((a - b).abs() <= 2.0 ** -7 * b.abs() + 1e-6).all()   # one bf16 ulp


@pytest.mark.parametrize("streams", [2, 3])
def test_layer_streams_identical_to_one_stream(streams):
    """decode() with the layers split over several streams gives bit-identical
    ids and outputs to the single-stream step (the layers are independent and
    each keeps its launch shape), step after step as the ring advances."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T, steps = 5, 8192, 4
    cfg = M12Config(max_model_len=T + 64)
    one = M12ModelRuntime(L, cfg, layer_streams=1)
    many = M12ModelRuntime(L, cfg, layer_streams=streams)
    hist = [workload.history(T, 300 + i) for i in range(L)]
    k = torch.stack([h[0] for h in hist]).cuda()
    v = torch.stack([h[1] for h in hist]).cuda()
    one.prefill(k, v)
    many.prefill(k, v)
    qs, ks, vs = workload.decode_inputs(steps, 11, layers=L)
    for s in range(steps):
        if s == steps - 1:
            many.layer_streams = 1           # a changed count takes effect on the next step
        q, kk, vv = qs[s].cuda(), ks[s].cuda(), vs[s].cuda()
        o1 = one.decode(q, kk, vv)
        o2 = many.decode(q, kk, vv)
        assert many._plan["nstreams"] == many.layer_streams
        assert one.last_n_selected == many.last_n_selected
        n = one.last_n_selected
        assert torch.equal(one.last_ids_dev[:, :, :n], many.last_ids_dev[:, :, :n])
        assert torch.equal(o1, o2)
        assert many.valid_len == one.valid_len


def test_layer_streams_in_the_stream_form():
    """With 16 layers the step's attention takes the stream form, whose
    partition of the segment list depends on the layers a launch holds: over
    two streams (two launches of 8 layers) the selected ids are identical and
    the outputs agree with the one-stream step to one bf16 ulp."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T, steps = 16, 8192, 3
    cfg = M12Config(max_model_len=T + 64)
    one = M12ModelRuntime(L, cfg, layer_streams=1)
    two = M12ModelRuntime(L, cfg, layer_streams=2)
    hist = [workload.history(T, 400 + i) for i in range(L)]
    k = torch.stack([h[0] for h in hist]).cuda()
    v = torch.stack([h[1] for h in hist]).cuda()
    one.prefill(k, v)
    two.prefill(k, v)
    assert one.core.decode_splits(one.core.effective_k(cfg.top_k_blocks)) == 0
    qs, ks, vs = workload.decode_inputs(steps, 13, layers=L)
    for s in range(steps):
        q, kk, vv = qs[s].cuda(), ks[s].cuda(), vs[s].cuda()
        a = one.decode(q, kk, vv).float().cpu()
        b = two.decode(q, kk, vv).float().cpu()
        n = one.last_n_selected
        assert torch.equal(one.last_ids_dev[:, :, :n], two.last_ids_dev[:, :, :n])
        assert ((a - b).abs() <= 2.0 ** -7 * b.abs() + 2e-6).all()


@pytest.mark.parametrize("quant", [False, True])
def test_decode_step_selection_with_tied_scores(quant):
    """nkv_decode_step's selection (protected blocks left unscored by the
    scorer, keys cleared by the attention launch) on layers whose scores tie
    heavily: random, half the blocks all-zero, all zero.  Ids equal the
    oracle's top-k of the oracle's scores over the same representatives, step
    after step (the keys start from zero every step)."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T = 3, 8192
    model = M12ModelRuntime(L, M12Config(max_model_len=T + 64, quant_history=quant))
    hist = [workload.history(T, 400 + i) for i in range(L)]
    model.prefill(torch.stack([h[0] for h in hist]).cuda(), torch.stack([h[1] for h in hist]).cuda())
    nb = model.nblocks_filled
    reps = model.store.reps[:, :, :nb]
    reps[1, :, ::2] = 0
    reps[2].zero_()
    prot = model.core.protected_blocks
    qs, ks, vs = workload.decode_inputs(3, 41, layers=L)
    for s in range(3):
        model.decode(qs[s].cuda(), ks[s].cuda(), vs[s].cuda())
        ids = model.last_ids_dev[:, 0, :model.last_n_selected].cpu()
        for i in range(L):
            s_or = O.block_scores(to_np(qs[s, i]), to_np(reps[i]), nb, 8)
            ids_or, _ = O.topk_blocks(s_or, prot, 32)
            assert ids[i].tolist() == ids_or.tolist(), f"step {s} layer {i}"
