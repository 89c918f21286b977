"""The rest of the reference's M12LayerRuntime call surface on the GPU:
_fused_attention over caller-packed K/V (m12_runtime.py:845-896), an
instance-level _gpu_select override steering prefill_chunk / decode /
verify_tokens (the reference's own tests force ids that way,
tests/test_m14_prefill_layout.py:61-90), the stage-profiling hooks
(:1130-1162) and the segmented-prefill adapter contract (:596-636)."""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import PREFILL_TOL, assert_close_bf16, to_np

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _rand(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _runtime(**kw):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    base = dict(block_size=64, r=4, recent_tokens=64, sink_tokens=64, top_k_blocks=6, max_model_len=2048)
    base.update(kw)
    return M12LayerRuntime(0, M12Config(**base))


@pytest.mark.parametrize("tq,s_len,causal_from,masked,tol", [
    (1, 2624, 2624, False, None),          # decode fast path
    (1, 2624, 5000, False, None),          # causal_from past the keys: all visible
    (3, 2627, 2624, True, None),           # few-query kernel, causal chunk + per-token mask
    (4, 700, 100, False, None),            # keys after causal_from + t hidden
    (200, 2824, 2624, False, PREFILL_TOL),   # matrix-core kernel
    (130, 1000, 870, True, PREFILL_TOL),     # matrix-core kernel with a per-token mask
])
def test_fused_attention_matches_oracle(tq, s_len, causal_from, masked, tol):
    rt = _runtime()
    g = torch.Generator().manual_seed(tq * 7 + s_len)
    q = _rand(g, tq, HQ, D)
    k = _rand(g, s_len, HKV, D, scale=D ** -0.5)
    v = _rand(g, s_len, HKV, D, scale=D ** -0.5)
    mask = None
    if masked:
        mask = torch.rand(tq, s_len, generator=g) < 0.3
        mask[:, 0] = False                   # every query keeps a key
    out = rt._fused_attention(q.cuda(), k.cuda(), v.cuda(), hist_len=s_len // 2, sink_len=64,
                              causal_from=causal_from, attn_mask=None if mask is None else mask.cuda())
    m = O.causal_mask(tq, s_len, causal_from, None if mask is None else mask.numpy())
    ref = O.attention_fp64(to_np(q), to_np(k), to_np(v), rt.cfg.scale, m)
    kw = {} if tol is None else tol
    worst = assert_close_bf16(to_np(out), ref, **kw)
    print(f"[_fused_attention tq={tq} S={s_len} causal_from={causal_from} mask={masked}] max |err| {worst:.2e}")


def test_fused_attention_rejects_bad_shapes():
    rt = _runtime()
    q = torch.zeros(2, HQ, D, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(10, HKV, D, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        rt._fused_attention(q, k[:, :4], k[:, :4], 0, 0, 10)
    with pytest.raises(ValueError):
        rt._fused_attention(q, k, k, 0, 0, 10, attn_mask=torch.zeros(2, 9, dtype=torch.bool, device="cuda"))
    with pytest.raises(ValueError):
        rt._fused_attention(q.float(), k, k, 0, 0, 10)


def _history(rt, T, seed):
    g = torch.Generator().manual_seed(seed)
    q0 = _rand(g, T, HQ, D)
    k0 = _rand(g, T, HKV, D, scale=D ** -0.5)
    v0 = _rand(g, T, HKV, D, scale=D ** -0.5)
    rt.prefill_first(q0.cuda(), k0.cuda(), v0.cuda())
    return g, k0, v0


def test_prefill_chunk_with_forced_ids_equals_full_history_attention():
    """Port of test_m14_prefill_layout.py:61-90 at the Qwen3-4B head shape:
    512 stored tokens (8 blocks; sink = block 0, recent = block 7), the
    selector forced to blocks 1-6, so the packed keys cover the whole
    history and the chunk's output equals plain causal attention over
    [history | chunk] (computed by _fused_attention and by the oracle)."""
    rt = _runtime()
    g, k0, v0 = _history(rt, 512, 7)
    rt._gpu_select = lambda _q: (torch.tensor([1, 2, 3, 4, 5, 6]), {"n_selected": 6})
    q1 = _rand(g, 256, HQ, D)
    k1 = _rand(g, 256, HKV, D, scale=D ** -0.5)
    v1 = _rand(g, 256, HKV, D, scale=D ** -0.5)
    actual = rt.prefill_chunk(q1.cuda(), k1.cuda(), v1.cuda(), torch.device("cuda"))
    kc, vc = torch.cat((k0, k1)).cuda(), torch.cat((v0, v1)).cuda()
    expected = rt._fused_attention(q1.cuda(), kc, vc, hist_len=512, sink_len=64, causal_from=512)
    ref = O.attention_fp64(to_np(q1), to_np(kc), to_np(vc), rt.cfg.scale, O.causal_mask(256, 768, 512))
    assert_close_bf16(to_np(actual), ref, **PREFILL_TOL)
    assert_close_bf16(to_np(expected), ref, **PREFILL_TOL)
    assert rt.valid_len == 768
    assert rt.last_prefill_block_ids.tolist() == [1, 2, 3, 4, 5, 6]


@pytest.mark.parametrize("bad", [[1, 8], [-1, 2], [3, 100]])
def test_selector_override_ids_outside_the_history_are_refused(bad):
    """Ids an override returns must name filled blocks (8 here): the kernels
    read blocks in place, so an id past the history or a negative one raises."""
    rt = _runtime()
    g, _, _ = _history(rt, 512, 17)
    rt._gpu_select = lambda _q, **kw: (torch.tensor(bad), {"n_selected": len(bad)})
    q1 = _rand(g, 64, HQ, D)
    kv = _rand(g, 64, HKV, D, scale=D ** -0.5)
    with pytest.raises(ValueError, match="outside"):
        rt.prefill_chunk(q1.cuda(), kv.cuda(), kv.cuda(), torch.device("cuda"))
    with pytest.raises(ValueError, match="outside"):
        rt.decode(q1[:1].cuda(), kv[:1].cuda(), kv[:1].cuda())


def test_decode_and_verify_honour_a_selector_override():
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    T = 8192
    cfg = M12Config(max_model_len=T + 64)
    rt = M12LayerRuntime(0, cfg)
    k, v, _, _ = workload.history(T, 61)
    rt.prefill_first(None, k.cuda(), v.cuda())
    ob = O.M12Oracle(O.OracleConfig())
    ob.store_kv(to_np(k), to_np(v), with_reps=False)
    forced = np.array([40, 3, 77, 12], dtype=np.int64)
    calls = []

    def fake_select(q, **kw):
        calls.append((tuple(q.shape), kw))
        return torch.tensor(forced), {"n_selected": len(forced)}

    rt._gpu_select = fake_select
    ob.select = lambda q, budget=None: (forced, None)
    qs, ks, vs = workload.decode_inputs(2, 62)
    for s in range(2):
        out = rt.decode(qs[s, 0].cuda(), ks[s, 0].cuda(), vs[s, 0].cuda())
        _, _, o_ref = ob.decode(to_np(qs[s, 0]), to_np(ks[s, 0]), to_np(vs[s, 0]))
        assert rt.last_block_ids.tolist() == forced.tolist()
        assert_close_bf16(to_np(out), o_ref)
    # the reference's decode call: the routing query [Hq, D] plus its keyword options
    assert calls[0][0] == (HQ, D)
    assert set(calls[0][1]) == {"dynamic", "budget", "use_graph", "use_static_mask", "use_relative"}
    # shared verify: the override receives the Tq queries
    g = torch.Generator().manual_seed(63)
    qv = _rand(g, 3, HQ, D)
    kv = _rand(g, 3, HKV, D, scale=D ** -0.5)
    vv = _rand(g, 3, HKV, D, scale=D ** -0.5)
    out = rt.verify_tokens(qv.cuda(), kv.cuda(), vv.cuda(), torch.device("cuda"))
    ids_or, o_ref = ob.verify_tokens(to_np(qv), to_np(kv), to_np(vv))
    assert ids_or.tolist() == forced.tolist()
    assert rt.last_verify_block_ids.tolist() == forced.tolist()
    assert_close_bf16(to_np(out), o_ref)
    assert calls[-1][0] == (3, HQ, D)


def test_cuda_stage_events_and_profile_ranges():
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    T = 4096
    rt = M12LayerRuntime(0, M12Config(max_model_len=T + 64))
    k, v, _, _ = workload.history(T, 71)
    rt.prefill_first(None, k.cuda(), v.cuda())
    qs, ks, vs = workload.decode_inputs(3, 72)
    rt.profile_cuda_stages = True
    rt.decode(qs[0, 0].cuda(), ks[0, 0].cuda(), vs[0, 0].cuda())
    torch.cuda.synchronize()
    # the names benchmark_m15_decode.py reads
    ms = {n: rt.cuda_stage_events[n][0].elapsed_time(rt.cuda_stage_events[n][1])
          for n in ("selector", "recent", "h2d_pack", "packed_attention")}
    assert all(t >= 0.0 for t in ms.values())
    assert ms["packed_attention"] > 0.0 and ms["selector"] > 0.0
    rt.profile_cuda_stages = False
    rt.profile_torch_stages = True
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        rt.decode(qs[1, 0].cuda(), ks[1, 0].cuda(), vs[1, 0].cuda())
    names = {e.name for e in prof.events()}
    assert {"m12.selector", "m12.packed_attention"} <= names
    rt.profile_torch_stages = False
    rt.profile_nsys_stages = True
    rt.decode(qs[2, 0].cuda(), ks[2, 0].cuda(), vs[2, 0].cuda())
    torch.cuda.synchronize()


class _PackingAdapter:
    """A prefill adapter honouring segmented_prefill_adapter.py's contract:
    prepare() receives (q, selected K, selected V, sink, recent, current)
    and attend() returns the chunk's output.  This one packs the segments and
    runs the runtime's own _fused_attention over them."""

    def __init__(self, rt):
        self.rt = rt
        self.seen = None

    def prepare(self, q, stage_k, stage_v, sink, recent, current):
        self.seen = (stage_k, stage_v, sink, recent, current)
        pk = torch.cat([stage_k, sink[0], recent[0], current[0]])
        pv = torch.cat([stage_v, sink[1], recent[1], current[1]])
        return q, pk, pv, pk.shape[0] - current[0].shape[0]

    def attend(self, inv):
        q, pk, pv, off = inv
        return self.rt._fused_attention(q, pk, pv, hist_len=0, sink_len=0, causal_from=off)


def test_prefill_adapter_receives_the_segments_and_its_output_is_returned():
    rt = _runtime(top_k_blocks=3)
    adapter = _PackingAdapter(rt)
    rt.cfg.prefill_adapter = adapter
    g, k0, v0 = _history(rt, 512, 81)
    rt._gpu_select = lambda _q: (torch.tensor([5, 2, 3]), {"n_selected": 3})
    q1 = _rand(g, 128, HQ, D)
    k1 = _rand(g, 128, HKV, D, scale=D ** -0.5)
    v1 = _rand(g, 128, HKV, D, scale=D ** -0.5)
    out = rt.prefill_chunk(q1.cuda(), k1.cuda(), v1.cuda(), torch.device("cuda"))
    sk, sv, sink, recent, cur = adapter.seen
    blocks = [k0[b * 64:(b + 1) * 64] for b in (5, 2, 3)]
    assert torch.equal(sk.cpu(), torch.cat(blocks))
    assert torch.equal(sink[0].cpu(), k0[:64]) and torch.equal(sink[1].cpu(), v0[:64])
    assert torch.equal(recent[0].cpu(), k0[448:]) and torch.equal(recent[1].cpu(), v0[448:])
    assert torch.equal(cur[0].cpu(), k1)
    keys = torch.cat(blocks + [k0[:64], k0[448:], k1])
    vals = torch.cat([v0[b * 64:(b + 1) * 64] for b in (5, 2, 3)] + [v0[:64], v0[448:], v1])
    ref = O.attention_fp64(to_np(q1), to_np(keys), to_np(vals), rt.cfg.scale,
                           O.causal_mask(128, keys.shape[0], keys.shape[0] - 128))
    assert_close_bf16(to_np(out), ref, **PREFILL_TOL)
    assert rt.valid_len == 640


def test_prefill_adapter_and_backend_errors():
    rt = _runtime(quant_history=True)
    rt.cfg.prefill_adapter = object()
    _history(rt, 256, 91)
    x = torch.zeros(64, HQ, D, dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros(64, HKV, D, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(AssertionError, match="incompatible"):
        rt.prefill_chunk(x, kv, kv, torch.device("cuda"))
    rt2 = _runtime(prefill_attention_backend="triton")
    _history(rt2, 256, 92)
    with pytest.raises(ValueError, match="unknown prefill attention backend"):
        rt2.prefill_chunk(x, kv, kv, torch.device("cuda"))


@pytest.mark.parametrize("tier", ["hbm", "host"])
def test_shipped_segmented_prefill_adapter_matches_oracle(tier):
    """The library's SegmentedPrefillAdapter (segmented_prefill_adapter.py:50-159)
    set as cfg.prefill_adapter and shared by two layers, as ModelRunner shares
    one adapter across all layers (model_runner.py:134-175): the runtime
    selects, prepare() packs [selected | sink | recent | chunk] into the
    shared scratch and attend() runs the packed matrix-core attention.  Ids
    exact and outputs against the oracle's prefill_chunk, over two chunks per
    layer; the HBM tier hands device tensors, the host tier pinned ones."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    from nanokv_amd.sparse.segmented_prefill_adapter import SegmentedPrefillAdapter
    adapter = SegmentedPrefillAdapter("flash_reuse", D ** -0.5, (HQ, HKV, D, torch.bfloat16))
    cfg = M12Config(max_model_len=8192, top_k_blocks=8, prefill_adapter=adapter, history_tier=tier)
    layers = [M12LayerRuntime(i, cfg) for i in range(2)]
    oracles = [O.M12Oracle(O.OracleConfig(top_k_blocks=8)) for _ in range(2)]
    g = torch.Generator().manual_seed(4242)
    for rt, ob in zip(layers, oracles):
        k0, v0 = _rand(g, 3000, HKV, D, scale=D ** -0.5), _rand(g, 3000, HKV, D, scale=D ** -0.5)
        rt.prefill_first(None, k0.cuda(), v0.cuda())
        ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    calls, biggest = 0, 0
    for T in (300, 129):
        for i, (rt, ob) in enumerate(zip(layers, oracles)):
            nb = rt.nblocks_filled
            ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])
            q = _rand(g, T, HQ, D)
            k, v = _rand(g, T, HKV, D, scale=D ** -0.5), _rand(g, T, HKV, D, scale=D ** -0.5)
            print(f"[adapter {tier}] layer {i} chunk of {T}", flush=True)
            out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda(), torch.device("cuda"))
            ids_or, o_ref = ob.prefill_chunk(to_np(q), to_np(k), to_np(v))
            assert rt.last_prefill_block_ids.tolist() == ids_or.tolist()
            worst = assert_close_bf16(to_np(out), o_ref, **PREFILL_TOL)
            print(f"  max |err| {worst:.3e}", flush=True)
            calls += 1
            biggest = max(biggest, 8 * 64 + 64 + 512 + T)
    st = adapter.stats()
    assert st["fa2_calls"] == calls and st["direct_calls"] == 0
    assert st["pack_capacity"] == biggest
    assert st["shared_scratch_bytes"] == 2 * biggest * HKV * D * 2


def test_shipped_adapter_rejects_pageable_staging_and_foreign_streams():
    """segmented_prefill_adapter.py:72-77, :100-101: pageable host staging and a
    stream other than the one the adapter was built on are refused."""
    from nanokv_amd.sparse.segmented_prefill_adapter import SegmentedPrefillAdapter
    adapter = SegmentedPrefillAdapter("flash_reuse", D ** -0.5, (HQ, HKV, D, torch.bfloat16))
    q = torch.zeros(40, HQ, D, dtype=torch.bfloat16, device="cuda")
    seg = torch.zeros(64, HKV, D, dtype=torch.bfloat16, device="cuda")
    cur = torch.zeros(40, HKV, D, dtype=torch.bfloat16, device="cuda")
    pageable = torch.zeros(128, HKV, D, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="selected CPU staging must be pinned"):
        adapter.prepare(q, pageable, pageable, (seg, seg), (seg, seg), (cur, cur))
    with pytest.raises(ValueError, match="inconsistent selected/current lengths"):
        adapter.prepare(q, seg, seg, (seg, seg), (seg, seg), (seg, seg))
    pinned = pageable.pin_memory()
    inv = adapter.prepare(q, pinned, pinned, (seg, seg), (seg, seg), (cur, cur))
    assert inv.packed[0].shape[0] == 128 + 64 + 64 + 40
    other = torch.cuda.Stream()
    with torch.cuda.stream(other):
        with pytest.raises(ValueError, match="one CUDA device/stream"):
            adapter.attend(inv)
    out = adapter.attend(inv)
    torch.cuda.synchronize()
    assert out.shape == (40, HQ, D) and torch.isfinite(out.float()).all()
