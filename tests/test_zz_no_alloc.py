"""nkv_decode_step_noalloc (scratch in the library's device array) against
nkv_decode_step with caller-allocated workspaces: two calls in a row, the
second on a smaller model (fewer layers, a shorter history, fewer splits),
then a third in the attention's stream form (splits 0), each compared bit
for bit with the allocating entry point on the same state (same kernels and
launch shapes, so ids and outputs are identical)."""

import ctypes

import pytest
import torch

from nanokv_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _model(L, T, seed):
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    model = M12ModelRuntime(L, M12Config(max_model_len=T + 64))
    hist = [workload.history(T, seed + i) for i in range(L)]
    model.prefill(torch.stack([h[0] for h in hist]).cuda(), torch.stack([h[1] for h in hist]).cuda())
    return model


def _both(model, q, k, v, splits):
    """The decode step of every layer through both entry points on one state.
    The ring write of the new token is the same in both calls (same slot,
    same data) and neither call reads that slot, so the second sees the
    first's inputs unchanged."""
    lib = _lib.load()
    core, st = model.core, model.store
    L, nb = model.num_layers, core.nblocks_filled
    req = model.cfg.top_k_blocks
    prot, n_prot = core.protected_dev()
    n = core.effective_k(req)
    w = core.decode_window()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    keys = torch.zeros(L * nb, dtype=torch.int32, device="cuda")
    part = torch.empty(max(1, st.decode_step_workspace_floats(L, splits, 1)), dtype=torch.float32, device="cuda")
    ids_a = torch.full((L, req), -7, dtype=torch.int32, device="cuda")
    ids_b = torch.full((L, req), -7, dtype=torch.int32, device="cuda")
    out_a = torch.empty_like(q)
    out_b = torch.empty_like(q)
    args = (st._desc_ref, 0, L, _ptr(q), _ptr(k), _ptr(v), nb, _ptr(prot), n_prot, req, n, w["sink_len"],
            w["write_slot"], w["ring_base"], w["rec_lo"], w["rec_len"], float(model.cfg.scale), splits)
    streams = (ctypes.c_void_p * 1)(stream)
    _lib.check(lib.nkv_decode_step(*args, _ptr(keys), _ptr(ids_a), _ptr(part), _ptr(out_a), 1, streams),
               "decode_step")
    _lib.check(lib.nkv_decode_step_noalloc(*args, _ptr(ids_b), _ptr(out_b), stream), "decode_step_noalloc")
    torch.cuda.synchronize()
    core.advance_decode()
    return n, ids_a, ids_b, out_a, out_b


def test_noalloc_decode_step_matches_the_allocating_entry_twice_in_a_row():
    from nanokv_amd import workload
    # call 1: 6 layers x 16K history, 5 splits; call 2: 2 layers x 4K, 3 splits;
    # call 3: 12 layers x 16K in the stream form (splits 0: one record per
    # wavefront and group in the partial region)
    for L, T, splits, seed in ((6, 16384, 5, 900), (2, 4096, 3, 950), (12, 16384, 0, 970)):
        model = _model(L, T, seed)
        qs, ks, vs = workload.decode_inputs(2, seed + 1, layers=L)
        for s in range(2):
            q, k, v = qs[s].cuda(), ks[s].cuda(), vs[s].cuda()
            n, ids_a, ids_b, out_a, out_b = _both(model, q, k, v, splits)
            print(f"[noalloc L={L} T={T} splits={splits} step {s}] ids {n} per layer", flush=True)
            assert torch.equal(ids_a[:, :n], ids_b[:, :n])
            assert bool((ids_b[:, :n] >= 0).all())
            assert torch.equal(out_a, out_b)


def test_noalloc_decode_step_rejects_oversized_calls():
    model = _model(1, 2048, 990)
    lib = _lib.load()
    st = model.store
    d = torch.zeros(64, dtype=torch.int32, device="cuda")
    # 2^20 blocks of score keys for one layer exceed the 262144-key region
    rc = lib.nkv_decode_step_noalloc(st._desc_ref, 0, 1, _ptr(d), _ptr(d), _ptr(d), 1 << 20, _ptr(d), 1, 32, 32,
                                     64, 0, 1, 0, 511, 1.0, 1, _ptr(d), _ptr(d), None)
    assert rc == _lib.NKV_ERR_ARG
    assert b"score keys" in lib.nkv_last_error()
