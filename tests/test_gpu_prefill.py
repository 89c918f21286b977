"""Many-query attention on the matrix cores (nkv_prefill_attend) vs the oracle.

The kernel replaces prefill_chunk's pack + bottom-right causal flash
attention (m12_runtime.py:560-651, :809-839).  Queries are the chunk's own
tokens; keys are [selected history | sink | previous recent | chunk (causal)].
Outputs are bf16 from fp32 accumulation with P rounded to bf16 for the
P.V product (as flash attention does); the bar is the fp64 oracle to about
one bf16 ulp and always within 2e-3 max-abs.  Selection must match exactly.

Covered: bf16 and both int8 layouts (dequantised to bf16 exactly as the
reference packs them), chunk lengths that are not multiples of the 32-token
query tile, multi-chunk prefill (store after attend), verify routed through
the same kernel with the lossless per-query mask and a rotated recent ring,
several layers in one launch, and the 4096-token chunk on a 32K history at
full size (sampled rows vs fp64, every row vs a float32 torch reference).
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import PREFILL_TOL, assert_close_bf16, to_np

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _pair(max_len, layout="channel_block", **kw):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    cfg = M12Config(max_model_len=max_len, quant_scale_layout=layout, **kw)
    rt = M12LayerRuntime(0, cfg)
    okw = {k: v for k, v in kw.items() if k in O.OracleConfig.__dataclass_fields__}
    if layout == "token":
        okw["quant_history"] = False   # the oracle is handed the GPU's dequantised history
    ob = O.M12Oracle(O.OracleConfig(**okw))
    return rt, ob


def _sync(rt, ob, token_layout):
    """Give the oracle the GPU-built representatives (and per-token int8 history)."""
    nb = rt.nblocks_filled
    assert nb == ob.nblocks_filled
    ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])
    if token_layout:
        st = rt.store
        kq = st.hist_k[0, :, :nb].cpu().numpy().astype(np.float32)
        vq = st.hist_v[0, :, :nb].cpu().numpy().astype(np.float32)
        ks = st.k_tscale[0, :, :nb * 64].cpu().float().numpy().reshape(8, nb, 64, 1)
        vs = st.v_tscale[0, :, :nb * 64].cpu().float().numpy().reshape(8, nb, 64, 1)
        ob.hist_k[:nb] = O.bf16_round(kq * ks).transpose(1, 2, 0, 3)
        ob.hist_v[:nb] = O.bf16_round(vq * vs).transpose(1, 2, 0, 3)


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8_token"])
def test_prefill_chunks_all_formats_match_oracle(fmt):
    """History 2000 tokens, then chunks of 33, 200 and 96 tokens (ragged query tiles)."""
    quant = fmt != "bf16"
    layout = "token" if fmt == "int8_token" else "channel_block"
    rt, ob = _pair(4096, layout=layout, quant_history=quant)
    k0, v0 = _rand((2000, 8, 128), 11, 0.09), _rand((2000, 8, 128), 12, 0.09)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    _sync(rt, ob, layout == "token")
    for i, T in enumerate((33, 200, 96)):
        print(f"[prefill {fmt}] chunk {i}: T={T}", flush=True)
        q = _rand((T, 32, 128), 20 + i)
        k, v = _rand((T, 8, 128), 30 + i, 0.09), _rand((T, 8, 128), 40 + i, 0.09)
        out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda())
        ids_or, o_ref = ob.prefill_chunk(to_np(q), to_np(k), to_np(v))
        _sync(rt, ob, layout == "token")
        assert rt.last_prefill_block_ids.tolist() == ids_or.tolist()
        worst = assert_close_bf16(to_np(out), o_ref, **PREFILL_TOL)
        print(f"  max |err| {worst:.3e}", flush=True)


def test_planted_query_chunk_attends_planted_blocks():
    """A chunk whose queries align with planted blocks selects them (selection drives attention)."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    k, v, q, planted = workload.history(8192, 77)
    rt = M12LayerRuntime(0, M12Config(max_model_len=8192 + 256))
    rt.prefill_first(None, k.cuda(), v.cuda())
    qc = q.unsqueeze(0).repeat(64, 1, 1)
    kc, vc = _rand((64, 8, 128), 78, 0.09), _rand((64, 8, 128), 79, 0.09)
    rt.prefill_chunk(qc.cuda(), kc.cuda(), vc.cuda())
    assert set(planted) <= set(rt.last_prefill_block_ids.tolist())


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8_token"])
def test_chunks_on_the_wide_few_query_kernel_match_oracle(fmt):
    """Chunks forced onto the few-query kernel (mfma_chunk_min_tokens above
    them): its wide form takes 32 query rows per group, so 7 tokens x 4 heads
    are one group, 100 tokens 13 groups and 37 tokens 5 with a ragged last
    one.  fp32 P.V, so bf16 history meets the tight bar; int8 history folds
    the K scale into the query operand / the logits (rel 2^-6)."""
    quant = fmt != "bf16"
    layout = "token" if fmt == "int8_token" else "channel_block"
    rt, ob = _pair(4096, layout=layout, quant_history=quant, mfma_chunk_min_tokens=10000)
    k0, v0 = _rand((2000, 8, 128), 13, 0.09), _rand((2000, 8, 128), 14, 0.09)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    _sync(rt, ob, layout == "token")
    tol = dict(rel=2.0 ** -6, abs_tol=2e-4) if quant else {}
    for i, T in enumerate((7, 100, 37)):
        print(f"[wide few-query {fmt}] chunk {i}: T={T}", flush=True)
        q = _rand((T, 32, 128), 90 + i)
        k, v = _rand((T, 8, 128), 93 + i, 0.09), _rand((T, 8, 128), 96 + i, 0.09)
        out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda())
        ids_or, o_ref = ob.prefill_chunk(to_np(q), to_np(k), to_np(v))
        _sync(rt, ob, layout == "token")
        assert rt.last_prefill_block_ids.tolist() == ids_or.tolist()
        worst = assert_close_bf16(to_np(out), o_ref, **tol)
        print(f"  max |err| {worst:.3e}", flush=True)


@pytest.mark.parametrize("kernel", ["mfma", "wide"])
@pytest.mark.parametrize("lossless", [False, True])
def test_verify_with_rotated_ring(lossless, kernel):
    """Verify chunks after decode steps rotated the ring, on the matrix-core
    kernel (forced) and on the few-query kernel's wide form (the automatic
    choice for 6 tokens x 4 heads)."""
    rt, ob = _pair(8192 + 128, top_k_blocks=16, mfma_chunk_min_tokens=1 if kernel == "mfma" else None)
    k0, v0 = _rand((8192, 8, 128), 50, 0.09), _rand((8192, 8, 128), 51, 0.09)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    ob.store_kv(to_np(k0), to_np(v0), with_reps=False)
    _sync(rt, ob, False)
    rt.verify_lossless = lossless
    for s in range(37):                      # ring_start moves to 37
        q, k, v = _rand((1, 32, 128), 60 + s), _rand((1, 8, 128), 160 + s, 0.09), _rand((1, 8, 128), 260 + s, 0.09)
        rt.decode(q.cuda(), k.cuda(), v.cuda())
        ob.decode(to_np(q), to_np(k), to_np(v))
    for rnd, accept in enumerate((4, 6)):
        tq = 6
        q = _rand((tq, 32, 128), 400 + rnd)
        k, v = _rand((tq, 8, 128), 410 + rnd, 0.09), _rand((tq, 8, 128), 420 + rnd, 0.09)
        out = rt.verify_tokens(q.cuda(), k.cuda(), v.cuda())
        ids_or, o_ref = ob.verify_tokens(to_np(q), to_np(k), to_np(v), lossless=lossless)
        assert rt.last_verify_block_ids.tolist() == ids_or.tolist()
        worst = assert_close_bf16(to_np(out), o_ref, **(PREFILL_TOL if kernel == "mfma" else {}))
        print(f"[verify {kernel} lossless={lossless}] round {rnd}: max |err| {worst:.3e}", flush=True)
        rt.commit_verified(accept)
        ob.commit_verified(accept)


def test_model_runtime_prefill_chunk_batches_layers():
    """M12ModelRuntime.prefill_chunk (one launch per stage for all layers) vs per-layer oracles."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T0, T = 3, 3000, 130
    cfg = M12Config(max_model_len=4096)
    model = M12ModelRuntime(L, cfg)
    hist = [workload.history(T0, 300 + i) for i in range(L)]
    kh = torch.stack([h[0] for h in hist]).cuda()
    vh = torch.stack([h[1] for h in hist]).cuda()
    model.prefill(kh, vh)
    nb0 = model.nblocks_filled
    q, k, v = workload.prefill_chunk_inputs(T, 5, layers=L)
    out = model.prefill_chunk(q.cuda(), k.cuda(), v.cuda()).cpu()
    for i in range(L):
        ob = O.M12Oracle(O.OracleConfig())
        ob.store_kv(to_np(hist[i][0]), to_np(hist[i][1]), with_reps=False)
        ob.reps[:, :nb0] = to_np(model.store.reps[i, :, :nb0])
        ids_or, o_ref = ob.prefill_chunk(to_np(q[i]), to_np(k[i]), to_np(v[i]))
        n = model.last_n_selected
        assert model.last_ids_dev[i, 0, :n].cpu().tolist() == ids_or.tolist()
        assert_close_bf16(to_np(out[i]), o_ref, **PREFILL_TOL)
    assert model.valid_len == T0 + T


def _torch_reference(q, pk, pv, off, scale):
    """float32 causal attention on the GPU: q [T, 32, D], pk/pv [S, 8, D]; query t sees keys < off + t + 1."""
    T, S = q.shape[0], pk.shape[0]
    out = torch.empty(T, 32, 128, dtype=torch.float32, device=q.device)
    cols = torch.arange(S, device=q.device)[None, :]
    rows = torch.arange(T, device=q.device)[:, None]
    mask = cols > rows + off                                           # [T, S]
    for h in range(8):
        kh = pk[:, h].float().contiguous()                            # [S, D]
        vh = pv[:, h].float().contiguous()
        qh = q[:, 4 * h:4 * h + 4].float().reshape(T * 4, 128).contiguous()
        logits = (qh @ kh.t().contiguous()).view(T, 4, S) * scale
        logits.masked_fill_(mask[:, None, :], float("-inf"))
        p = torch.softmax(logits, dim=-1)
        out[:, 4 * h:4 * h + 4] = (p.view(T * 4, S) @ vh).view(T, 4, 128)
    return out


def test_prefill_4096_chunk_on_32k_history_full_size():
    """The 4096-token chunk against a 32K bf16 history (32 selected blocks + sink + recent)."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    T0, T = 32768, 4096
    cfg = M12Config(max_model_len=T0 + T)
    rt = M12LayerRuntime(0, cfg)
    k0, v0, _, _ = workload.history(T0, 2024)
    rt.prefill_first(None, k0.cuda(), v0.cuda())
    q, k, v = workload.prefill_chunk_inputs(T, 2024)
    q, k, v = q[0], k[0], v[0]
    print("[prefill 32K] running the 4096-token chunk", flush=True)
    out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda())
    torch.cuda.synchronize()
    ids = rt.last_prefill_block_ids
    # selection: same representatives -> the oracle's Top-32 of the query-mean summary
    nb0 = T0 // 64
    reps = to_np(rt.reps_gpu[:, :nb0])
    qs = O.query_summaries(to_np(q), 1)
    prot = O.protected_blocks_after_store(nb0, 512, 64)
    ids_or, _ = O.select_blocks(qs, reps, nb0, 8, prot, 32)
    assert ids.tolist() == ids_or.tolist()
    # packed keys as the reference builds them: [selected | sink | last 512 of history | chunk]
    kb = k0.view(nb0, 64, 8, 128)
    vb = v0.view(nb0, 64, 8, 128)
    idx = torch.as_tensor(ids_or, dtype=torch.int64)
    _, roff, rlen = O.prefill_recent_slice(T0, 64, 512)
    pk = torch.cat([kb[idx].reshape(-1, 8, 128), k0[:64], k0[T0 - 512 + roff:T0 - 512 + roff + rlen], k])
    pv = torch.cat([vb[idx].reshape(-1, 8, 128), v0[:64], v0[T0 - 512 + roff:T0 - 512 + roff + rlen], v])
    off = pk.shape[0] - T
    assert off == 32 * 64 + 64 + 512
    got = out.float().cpu()
    # every row vs a float32 torch reference
    ref32 = _torch_reference(q.cuda(), pk.cuda(), pv.cuda(), off, cfg.scale).cpu()
    err = (got - ref32).abs().max().item()
    print(f"[prefill 32K] max |err| vs fp32 torch over all rows: {err:.3e}", flush=True)
    assert err <= 2e-3
    # sampled rows (first / tile edges / diagonal / last) vs the fp64 oracle
    rows = sorted({0, 1, 31, 32, 63, 64, 65, 127, 128, 1000, 2047, 2048, 3071, 4000, 4094, 4095})
    pkn, pvn, qn = to_np(pk), to_np(pv), to_np(q)
    for t in rows:
        o_ref = O.attention_fp64(qn[t:t + 1], pkn[:off + t + 1], pvn[:off + t + 1], cfg.scale)
        assert_close_bf16(to_np(out[t:t + 1]), o_ref, **PREFILL_TOL)


@pytest.mark.parametrize("T0,T,tile,top_k,model", [
    (4096, 300, 64, 8, False),     # 5 tiles, the last one short
    (8192, 512, 64, 32, False),    # 8 full tiles
    (8192, 512, 128, 32, True),    # all layers at once, 4 tiles of 128
    (8192, 600, 96, 32, False),    # 192-column kernel: two 48-token workgroups per tile, the last tile short
    (8192, 768, 192, 16, True),    # 192-column kernel, all layers, four workgroups per tile
])
def test_prefill_per_tile_selection_matches_oracle(T0, T, tile, top_k, model):
    """prefill_selection="tile": one Top-K per tile of queries from the tile's
    query mean; each tile attends its own blocks (oracle prefill_chunk_tiled)."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12LayerRuntime, M12ModelRuntime
    cfg = M12Config(max_model_len=T0 + T + 64, top_k_blocks=top_k, prefill_selection="tile",
                    prefill_selection_tile=tile)
    L = 3 if model else 1
    hist = [workload.history(T0, 700 + i) for i in range(L)]
    q, k, v = workload.prefill_chunk_inputs(T, 71, layers=L)
    if model:
        rt = M12ModelRuntime(L, cfg)
        rt.prefill(torch.stack([h[0] for h in hist]).cuda(), torch.stack([h[1] for h in hist]).cuda())
        reps = [rt.store.reps[i] for i in range(L)]
        out = rt.prefill_chunk(q.cuda(), k.cuda(), v.cuda())
        ids_all = rt.last_ids_dev[:, :, :rt.last_n_selected].cpu()
    else:
        rt = M12LayerRuntime(0, cfg)
        rt.prefill_first(None, hist[0][0].cuda(), hist[0][1].cuda())
        reps = [rt.reps_gpu]
        out = rt.prefill_chunk(q[0].cuda(), k[0].cuda(), v[0].cuda(), torch.device("cuda")).unsqueeze(0)
        ids_all = rt.last_prefill_block_ids.unsqueeze(0)
    assert ids_all.shape[1] == -(-T // tile)
    for i in range(L):
        ob = O.M12Oracle(O.OracleConfig(top_k_blocks=top_k))
        ob.store_kv(to_np(hist[i][0]), to_np(hist[i][1]), with_reps=False)
        nb = ob.nblocks_filled
        ob.reps[:, :nb] = to_np(reps[i][:, :nb])
        ids_or, o_ref = ob.prefill_chunk_tiled(to_np(q[i]), to_np(k[i]), to_np(v[i]), tile)
        assert ids_all[i].tolist() == ids_or.tolist(), f"layer {i}: tile ids differ"
        assert_close_bf16(to_np(out[i]), o_ref, **PREFILL_TOL)


def test_prefill_per_tile_selection_full_size_36_layers():
    """The launch `bench.py --workload prefill --prefill-selection tile` times:
    a 4096-token chunk of each of 36 layers against its 32K bf16 history, one
    Top-32 per 64-query tile (64 tiles per layer), then the matrix-core
    attention with each tile's own blocks.  Sampled layers: per-tile ids exact
    against the oracle's selection over the GPU representatives, every row
    against a float32 torch reference of the tile's packed keys, and sampled
    rows (tile edges, the diagonal, the last row) against the fp64 oracle."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    L, T0, T, tile, K, seed = 36, 32768, 4096, 64, 32, 1234
    cfg = M12Config(max_model_len=T0 + T, top_k_blocks=K, prefill_selection="tile",
                    prefill_selection_tile=tile)
    model = M12ModelRuntime(L, cfg)
    kh = torch.empty(L, T0, 8, 128, dtype=torch.bfloat16, device="cuda")
    vh = torch.empty_like(kh)
    for i in range(L):
        k, v, _, _ = workload.history(T0, seed + i, device="cuda")
        kh[i].copy_(k)
        vh[i].copy_(v)
    model.prefill(kh, vh)
    q, k, v = workload.prefill_chunk_inputs(T, seed, device="cuda", layers=L)
    core = model.core
    print("[tile prefill 36 x 32K] selection + attention launch", flush=True)
    ids, n = core.select_tiles(q, K, tile)
    out, _, _ = core.chunk_attend_tiled(q, k, v, ids, tile, n)
    torch.cuda.synchronize()
    nb0 = T0 // 64
    assert n == K and ids.shape[:2] == (L, T // tile)
    prot = O.protected_blocks_after_store(nb0, cfg.recent_tokens, 64)
    _, roff, rlen = O.prefill_recent_slice(T0, cfg.sink_tokens, cfg.recent_tokens)
    off = K * 64 + cfg.sink_tokens + rlen
    for layer in (0, 17, 35):
        reps = to_np(model.store.reps[layer, :, :nb0])
        qn = to_np(q[layer])
        ids_l = ids[layer].cpu()
        kb = kh[layer].view(nb0, 64, 8, 128)
        vb = vh[layer].view(nb0, 64, 8, 128)
        prior_k = torch.cat([kh[layer, :cfg.sink_tokens], kh[layer, T0 - 512 + roff:T0 - 512 + roff + rlen]])
        prior_v = torch.cat([vh[layer, :cfg.sink_tokens], vh[layer, T0 - 512 + roff:T0 - 512 + roff + rlen]])
        worst32 = 0.0
        for ti in range(T // tile):
            t0, t1 = ti * tile, (ti + 1) * tile
            qs = O.query_summaries(qn[t0:t1], 1)
            ids_or, _ = O.select_blocks(qs, reps, nb0, 8, prot, K)
            assert ids_l[ti, :n].tolist() == ids_or.tolist(), f"layer {layer} tile {ti}: ids differ"
            idx = ids_l[ti, :n].to("cuda", torch.int64)
            pk = torch.cat([kb[idx].reshape(-1, 8, 128), prior_k, k[layer, :t1]])
            pv = torch.cat([vb[idx].reshape(-1, 8, 128), prior_v, v[layer, :t1]])
            ref32 = _torch_reference(q[layer, t0:t1], pk, pv, off + t0, cfg.scale)
            worst32 = max(worst32, (out[layer, t0:t1].float() - ref32).abs().max().item())
            rows = [r for r in (0, 63, 64, 2047, 2048, 4095) if t0 <= r < t1]
            if rows:
                pkn, pvn = to_np(pk), to_np(pv)
                for r in rows:
                    o_ref = O.attention_fp64(qn[r:r + 1], pkn[:off + r + 1], pvn[:off + r + 1], cfg.scale)
                    assert_close_bf16(to_np(out[layer, r:r + 1]), o_ref, **PREFILL_TOL)
        print(f"[tile prefill 36 x 32K] layer {layer}: 64 tiles' ids exact, "
              f"max |err| vs fp32 torch {worst32:.3e}", flush=True)
        assert worst32 <= 2e-3
