"""The splits-0 forms against the split form and the oracle: the 4-row
attention kernel's stream form, and the wide few-query kernel's tiered plan.

The batched decode step takes the stream form once a launch holds >= 4096
segments: one resident round of wavefronts, each attending an equal run of
the launch's (layer, KV head, segment) list and writing one partial record
per (layer, KV head) it touches, merged by the split-merge kernel.  These
cases drive it beyond the 36-layer Qwen3-4B headline (tests/test_gpu_headline.py):
GQA ratios 1, 2 and 4, budgets that leave an odd number of history segments,
both int8 scale layouts, short windows (sink and recent not yet full), and
history ids outside the history (which attend nothing).

The split and stream forms add the same terms in different orders, so their
outputs agree to about one bf16 ulp; selected ids are identical, and sampled
layers match the fp64 oracle (m12_runtime.py:1141-1346) as in the other
decode tests.
"""

import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import assert_close_bf16, to_np

pytestmark = pytest.mark.gpu

D = 128


def _models(L, T, hq, hkv, top_k, quant, layout, seed):
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    kw = dict(max_model_len=T + 64, num_heads=hq, num_kv_heads=hkv, top_k_blocks=top_k,
              quant_history=quant, quant_scale_layout=layout)
    stream = M12ModelRuntime(L, M12Config(**kw))
    split = M12ModelRuntime(L, M12Config(attend_splits=3, **kw))
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(L, T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    v = (torch.randn(L, T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    stream.prefill(k.cuda(), v.cuda())
    split.prefill(k.cuda(), v.cuda())
    return stream, split, k, v, g


# (L, T, Hq, Hkv, top_k, int8 layout or None, seed)
CASES = [
    (16, 8192, 32, 8, 32, None, 31),            # G = 4, the headline shape at 8K
    (16, 8192, 16, 8, 27, None, 32),            # G = 2, an odd history count
    (24, 4096, 8, 8, 13, None, 33),             # G = 1
    (16, 8192, 32, 8, 31, "channel_block", 34),  # int8, per-block scales
    (16, 8192, 32, 8, 32, "token", 35),          # int8, per-token scales
]


@pytest.mark.parametrize("L,T,hq,hkv,top_k,layout,seed", CASES)
def test_stream_form_matches_split_form_and_oracle(L, T, hq, hkv, top_k, layout, seed):
    quant = layout is not None
    print(f"case L={L} T={T} Hq={hq} Hkv={hkv} k={top_k} int8={layout}", flush=True)
    stream, split, k, v, g = _models(L, T, hq, hkv, top_k, quant, layout or "channel_block", seed)
    n = stream.core.effective_k(top_k)
    assert stream.core.decode_splits(n) == 0, "the case must take the stream form"
    assert split.core.decode_splits(n) == 3
    sampled = (0, L - 1)
    oracles = {}
    for i in sampled:
        if layout == "token":
            continue   # the per-token layout's oracle check lives in the headline / decode tests
        ob = O.M12Oracle(O.OracleConfig(num_heads=hq, num_kv_heads=hkv, top_k_blocks=top_k, quant_history=quant))
        ob.store_kv(to_np(k[i]), to_np(v[i]), with_reps=False)
        nb = stream.nblocks_filled
        ob.reps[:, :nb] = to_np(stream.store.reps[i, :, :nb])
        oracles[i] = ob
    worst = 0.0
    for s in range(3):
        q = torch.randn(L, 1, hq, D, generator=g).bfloat16()
        kn = (torch.randn(L, 1, hkv, D, generator=g) * D ** -0.5).bfloat16()
        vn = (torch.randn(L, 1, hkv, D, generator=g) * D ** -0.5).bfloat16()
        a = stream.decode(q.cuda(), kn.cuda(), vn.cuda()).float().cpu()
        b = split.decode(q.cuda(), kn.cuda(), vn.cuda()).float().cpu()
        ns = stream.last_n_selected
        assert ns == split.last_n_selected
        assert torch.equal(stream.last_ids_dev[:, 0, :ns].cpu(), split.last_ids_dev[:, 0, :ns].cpu())
        assert ((a - b).abs() <= 2.0 ** -7 * b.abs() + 2e-6).all(), f"step {s}: stream and split forms differ"
        for i, ob in oracles.items():
            ids_or, _, o_ref = ob.decode(to_np(q[i]), to_np(kn[i]), to_np(vn[i]))
            assert stream.last_ids_dev[i, 0, :ns].cpu().tolist() == ids_or.tolist(), f"step {s} layer {i}: ids"
            rel, abs_tol = (2.0 ** -6, 2e-4) if quant else (2.0 ** -7, 2e-5)
            worst = max(worst, assert_close_bf16(a[i].numpy(), o_ref, rel=rel, abs_tol=abs_tol))
    print(f"  stream vs oracle max |err| {worst:.3e}", flush=True)


def test_stream_form_short_window_and_foreign_ids():
    """nkv_attend with splits 0 over a short history (sink and recent not yet
    full), with some ids outside [0, cap) and an odd id count: the same output
    as the one-split form (no merge) to one bf16 ulp; ids outside the history
    attend nothing, so replacing them by -1 changes nothing."""
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T, hq, hkv = 40, 300, 32, 8
    cfg = M12Config(max_model_len=4096, num_heads=hq, num_kv_heads=hkv, top_k_blocks=8)
    model = M12ModelRuntime(L, cfg)
    g = torch.Generator().manual_seed(41)
    k = (torch.randn(L, T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    v = (torch.randn(L, T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    model.prefill(k.cuda(), v.cuda())
    core, st = model.core, model.store
    w = core.decode_window()
    nb = model.nblocks_filled
    n_hist = 5
    ids = torch.randint(0, nb, (L, n_hist), generator=g, dtype=torch.int32)
    ids[::3, 1] = -1                     # outside the history: attends nothing
    ids[1::4, 3] = st.cap_blocks + 7
    q = torch.randn(L, 1, hq, D, generator=g).bfloat16().cuda()
    kn = (torch.randn(L, 1, hkv, D, generator=g) * D ** -0.5).bfloat16().cuda()
    vn = (torch.randn(L, 1, hkv, D, generator=g) * D ** -0.5).bfloat16().cuda()
    ids_d = ids.cuda()
    outs = {}
    for splits in (0, 1):
        part = torch.empty(max(1, st.attend_workspace_floats(L, 1, splits)), dtype=torch.float32, device="cuda")
        out = torch.empty_like(q)
        # write_slot -1: the new token is only attended (this call must not move the ring)
        st.attend(0, q, kn, vn, 1, -1, ids_d, n_hist, n_hist, None, w["sink_len"], w["ring_base"], w["rec_lo"],
                  w["rec_len"], cfg.scale, splits, part, out)
        torch.cuda.synchronize()
        outs[splits] = out.float().cpu()
    a, b = outs[0], outs[1]
    assert torch.isfinite(a).all()
    assert ((a - b).abs() <= 2.0 ** -7 * b.abs() + 2e-6).all()
    # ids outside the history are the same as -1
    ids2 = ids.clone()
    ids2[ids2 >= st.cap_blocks] = -1
    part = torch.empty(max(1, st.attend_workspace_floats(L, 1, 0)), dtype=torch.float32, device="cuda")
    out2 = torch.empty_like(q)
    st.attend(0, q, kn, vn, 1, -1, ids2.cuda(), n_hist, n_hist, None, w["sink_len"], w["ring_base"], w["rec_lo"],
              w["rec_len"], cfg.scale, 0, part, out2)
    torch.cuda.synchronize()
    assert torch.equal(out2.float().cpu(), a)
    # the stream form is refused where it does not apply: 16 query rows (tq = 4)
    q4 = torch.randn(L, 4, hq, D, generator=g).bfloat16().cuda()
    with pytest.raises(ValueError, match="stream form"):
        st.attend(0, q4, None, None, 0, -1, ids_d, n_hist, n_hist, None, w["sink_len"], w["ring_base"], w["rec_lo"],
                  w["rec_len"], cfg.scale, 0, part, torch.empty_like(q4))


@pytest.mark.parametrize("L,T,top_k,quant,seed", [
    (16, 4096, 16, False, 51),    # 128 groups: 7 splits for the first 73, 9 for the other 55
    (40, 4096, 16, True, 52),     # 320 groups: 3 splits for the first 170, 3 for the rest
    (56, 2048, 8, False, 53),     # 448 groups: 2 splits for the first 256, 2 for the rest
    (72, 2048, 8, True, 54),      # 576 groups fill the 512 slots: one workgroup per group
])
def test_wide_plan_matches_split_form_and_oracle(L, T, top_k, quant, seed):
    """Lossless verify (6 draft tokens x G = 4: 24 rows, the wide kernel)
    with the runtime's automatic choice (splits 0, the tiered plan) against
    the same round at 3 uniform splits: identical unions, outputs within one
    bf16 ulp; a sampled layer against the fp64 oracle (m12_runtime.py:656-758)."""
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    hq, hkv, tq = 32, 8, 6
    kw = dict(max_model_len=T + 64, num_heads=hq, num_kv_heads=hkv, top_k_blocks=top_k, quant_history=quant)
    plan = M12ModelRuntime(L, M12Config(**kw))
    split = M12ModelRuntime(L, M12Config(attend_splits=3, **kw))
    assert plan.core._splits(top_k + 10, 1, tq * hq // hkv) == 0, "the case must take the tiered plan"
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(L, T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    v = (torch.randn(L, T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    plan.prefill(k.cuda(), v.cuda())
    split.prefill(k.cuda(), v.cuda())
    i = L - 1
    ob = O.M12Oracle(O.OracleConfig(num_heads=hq, num_kv_heads=hkv, top_k_blocks=top_k, quant_history=quant))
    ob.store_kv(to_np(k[i]), to_np(v[i]), with_reps=False)
    nb = plan.nblocks_filled
    ob.reps[:, :nb] = to_np(plan.store.reps[i, :, :nb])
    q = torch.randn(L, tq, hq, D, generator=g).bfloat16()
    kn = (torch.randn(L, tq, hkv, D, generator=g) * D ** -0.5).bfloat16()
    vn = (torch.randn(L, tq, hkv, D, generator=g) * D ** -0.5).bfloat16()
    print(f"case L={L} T={T} k={top_k} int8={quant}", flush=True)
    a = plan.verify(q.cuda(), kn.cuda(), vn.cuda(), lossless=True).float().cpu()
    b = split.verify(q.cuda(), kn.cuda(), vn.cuda(), lossless=True).float().cpu()
    assert torch.equal(plan.last_union_count_dev.cpu(), split.last_union_count_dev.cpu())
    assert torch.equal(plan.last_union_dev.cpu(), split.last_union_dev.cpu())
    assert ((a - b).abs() <= 2.0 ** -7 * b.abs() + 2e-6).all(), "tiered plan and split form differ"
    ids_or, o_ref = ob.verify_tokens(to_np(q[i]), to_np(kn[i]), to_np(vn[i]), lossless=True)
    cnt = int(plan.last_union_count_dev[i])
    assert plan.last_union_dev[i, :cnt].cpu().tolist() == ids_or.tolist()
    rel, abs_tol = (2.0 ** -6, 2e-4) if quant else (2.0 ** -7, 2e-5)
    worst = assert_close_bf16(a[i].numpy(), o_ref, rel=rel, abs_tol=abs_tol)
    print(f"  plan vs oracle max |err| {worst:.3e}", flush=True)


def test_attend_marks_bracket_the_attention_kernel():
    """nkv_set_attend_marks: with marks set, the stream-form decode attention
    records `before` right before the attention kernel and `after` right after
    it, ahead of the merge (so start <= before <= after <= end on the stream,
    both spans positive), and the output is bit-identical to the same call
    without marks; after clearing them no later launch records them again."""
    from nanokv_amd import _lib
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T = 16, 8192
    model = M12ModelRuntime(L, M12Config(max_model_len=T + 64, top_k_blocks=32))
    g = torch.Generator().manual_seed(61)
    k = (torch.randn(L, T, 8, D, generator=g) * D ** -0.5).bfloat16()
    v = (torch.randn(L, T, 8, D, generator=g) * D ** -0.5).bfloat16()
    model.prefill(k.cuda(), v.cuda())
    core = model.core
    q = torch.randn(L, 1, 32, D, generator=g).bfloat16().cuda()
    kn = (torch.randn(L, 1, 8, D, generator=g) * D ** -0.5).bfloat16().cuda()
    vn = (torch.randn(L, 1, 8, D, generator=g) * D ** -0.5).bfloat16().cuda()
    ids, _, n = model.select(q)
    assert core.decode_splits(n) == 0, "the case must take the stream form"
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]   # start, before, after, end
    for e in ev:
        e.record()
    torch.cuda.synchronize()
    outs = []
    for mark in (True, False):
        if mark:
            _lib.set_attend_marks(ev[1].cuda_event, ev[2].cuda_event)
        try:
            ev[0].record()
            o, _, _ = core.decode_attend(q, kn, vn, ids, ids.shape[-1], n, advance=False)
            ev[3].record()
        finally:
            _lib.set_attend_marks(None, None)
        torch.cuda.synchronize()
        outs.append(o.clone())
        if mark:
            spans = [ev[j].elapsed_time(ev[j + 1]) for j in range(3)]
            assert spans[0] >= 0 and spans[1] > 0 and spans[2] > 0, spans
            t_after = spans[2]
    assert torch.equal(outs[0], outs[1])
    # cleared: the second call did not record the marks again (the span from
    # the first call's `after` to the second call's end covers that call)
    assert ev[2].elapsed_time(ev[3]) > t_after
