"""The attention-layer entry point on the GPU kernels.

`nanokv_amd.attention.Attention` routes q/k/v as the reference's
Attention.forward does in sparse mode (nanovllm/layers/attention.py:64-99)
and `attach_m12_runtimes` wires one runtime per layer over one shared HBM
store (nanovllm/engine/model_runner.py:125-183).  A two-layer stand-in model
is driven through a whole sequence: the first prefill chunk (dense causal
attention within the chunk, which the reference hands to flash-attention), a
second chunk (sparse chunked prefill), decode steps and a verify round that
commits part of its tokens.

Checks: the first chunk against fp64 causal attention within the chunk (the
oracle) under the rounding bound of bf16 probabilities and bf16 outputs (see
_assert_within_bf16_bound); every later output and selection
bit-identical to a standalone M12LayerRuntime given the same calls (the
routing and the shared store add nothing to the arithmetic); the reference's
decode assertions (one token, no paged block tables).
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import to_np

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).cuda()


def _assert_within_bf16_bound(o, q, k, v, scale, mask):
    """|o - exact| <= u (|exact| + sum_s p_s |v_s|) elementwise, u = 2^-8 (bf16 round-to-nearest).

    The matrix-core kernel rounds the probabilities to bf16 for P.V (as the
    reference's flash-attention does) and rounds the output to bf16; the
    first rounding moves the output by at most u sum p|v| / l, the second by
    at most u |o|.  The fp32 exponentials and accumulation add a few 2^-24
    relative, covered by the 1% and 1e-5 slack.  In the first rows of a
    causal chunk the outputs are O(1), so the output rounding alone exceeds
    a flat 2e-3 absolute bar (for any bf16-output kernel); the bound is per
    element instead.  A wrong mask, key or value breaks it by orders of
    magnitude.
    """
    ref = O.attention_fp64(q, k, v, scale, mask)
    mag = O.attention_fp64(q, k, np.abs(v), scale, mask)   # sum_s p_s |v_s| with p normalised
    err = np.abs(np.asarray(o, dtype=np.float64) - ref)
    bound = 2.0 ** -8 * (np.abs(ref) + mag) * 1.01 + 1e-5
    assert np.isfinite(o).all()
    bad = err > bound
    assert not bad.any(), (f"{int(bad.sum())} outputs outside the bf16 bound; worst ratio "
                           f"{float((err / bound).max()):.3f}")
    return float((err / bound).max())


def _qkv(t, seed):
    return (_rand((t, HQ, D), seed), _rand((t, HKV, D), seed + 1, D ** -0.5),
            _rand((t, HKV, D), seed + 2))


class _TwoLayers(torch.nn.Module):
    def __init__(self, scale):
        super().__init__()
        from nanokv_amd.attention import Attention
        self.a0 = Attention(HQ, D, scale, HKV)
        self.a1 = Attention(HQ, D, scale, HKV)


def test_attention_layer_routes_a_whole_sequence():
    from nanokv_amd.attention import attach_m12_runtimes, reset_context, set_context
    from nanokv_amd.sparse import M12Config, M12LayerRuntime

    cfg = M12Config(max_model_len=4096, top_k_blocks=8)
    scale = D ** -0.5
    model = _TwoLayers(scale)
    rts = attach_m12_runtimes(model, cfg)
    layers = [model.a0, model.a1]
    assert [m.layer_id for m in layers] == [0, 1]
    assert rts[0].store is rts[1].store and [m.sparse_rt for m in layers] == rts
    assert all(m.k_cache.numel() == 0 and m.v_cache.numel() == 0 for m in layers)
    solo = [M12LayerRuntime(i, cfg) for i in range(2)]
    T1, T2 = 700, 300   # neither a multiple of the 64-token block
    try:
        print("first chunk (dense causal)", flush=True)
        set_context(True, max_seqlen_q=T1, max_seqlen_k=T1)
        for i, layer in enumerate(layers):
            q, k, v = _qkv(T1, 100 + 10 * i)
            o = layer(q, k, v)
            ratio = _assert_within_bf16_bound(to_np(o), to_np(q), to_np(k), to_np(v), scale,
                                              O.causal_mask(T1, T1, 0))
            print(f"layer {i}: worst error / bound = {ratio:.3f}", flush=True)
            solo[i].prefill_first(q, k, v)
            assert layer.sparse_rt.prefill_len == solo[i].prefill_len == T1
            assert layer.sparse_rt.nblocks_filled == solo[i].nblocks_filled
            assert torch.equal(layer.sparse_rt.reps_gpu, solo[i].reps_gpu)

        print("second chunk (sparse chunked prefill)", flush=True)
        set_context(True, max_seqlen_q=T2, max_seqlen_k=T1 + T2)
        for i, layer in enumerate(layers):
            q, k, v = _qkv(T2, 200 + 10 * i)
            o = layer(q, k, v)
            assert torch.equal(o, solo[i].prefill_chunk(q, k, v, q.device))
            assert torch.equal(layer.sparse_rt.last_prefill_block_ids, solo[i].last_prefill_block_ids)

        print("decode", flush=True)
        set_context(False)
        for step in range(3):
            for i, layer in enumerate(layers):
                q, k, v = _qkv(1, 300 + 10 * step + i)
                o = layer(q, k, v)
                assert torch.equal(o, solo[i].decode(q, k, v, q.device))
                assert torch.equal(layer.sparse_rt.last_block_ids, solo[i].last_block_ids)
                assert layer.sparse_rt.valid_len == solo[i].valid_len == T1 + T2 + step + 1

        print("verify + commit", flush=True)
        for i, layer in enumerate(layers):
            layer.sparse_rt.verify_mode = solo[i].verify_mode = True
            q, k, v = _qkv(5, 400 + 10 * i)
            o = layer(q, k, v)
            assert torch.equal(o, solo[i].verify_tokens(q, k, v, q.device))
            layer.sparse_rt.commit_verified(3)
            solo[i].commit_verified(3)
            layer.sparse_rt.verify_mode = solo[i].verify_mode = False
        q, k, v = _qkv(1, 500)
        assert torch.equal(model.a0(q, k, v), solo[0].decode(q, k, v, q.device))

        print("decode assertions", flush=True)
        q, k, v = _qkv(2, 600)
        with pytest.raises(AssertionError, match="single query token"):
            model.a1(q, k, v)
        set_context(False, block_tables=torch.zeros(1, 1, dtype=torch.int32))
        q, k, v = _qkv(1, 700)
        with pytest.raises(AssertionError, match="block tables"):
            model.a1(q, k, v)
    finally:
        reset_context()
