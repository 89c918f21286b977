"""The exact launch the decode benchmark times, checked against the oracle.

M12ModelRuntime over 36 layers of 32768-token histories (512 blocks each)
decodes through nkv_decode_step with the automatic attention split choice
(the stream form, 0, in every history format), the same seeds and inputs as
bench.py's default line and its int8 / int8_token lines.  On four sampled
layers the selected ids must equal the oracle's (value and order) and the
outputs must match the fp64 oracle to about one bf16 ulp at every step
(m12_runtime.py:1141-1346).
"""

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import assert_close_bf16, to_np

pytestmark = pytest.mark.gpu

L, T, SEED, STEPS = 36, 32768, 2024, 3
SAMPLED = (0, 13, 26, 35)


def _oracle_for_layer(model, i, kh, vh, quant, layout):
    """The oracle of layer i, holding the GPU's representatives.  For the
    per-token fp16-scale layout it attends the dequantised history the GPU
    stored, bf16(code * scale); the codes and scales themselves are checked
    bit-exact against the oracle's quantiser by the single-layer per-token
    decode test."""
    st = model.store
    nb = model.nblocks_filled
    token = quant and layout == "token"
    ob = O.M12Oracle(O.OracleConfig(quant_history=quant and not token))
    ob.store_kv(to_np(kh[i]), to_np(vh[i]), with_reps=False)
    ob.reps[:, :nb] = to_np(st.reps[i, :, :nb])
    if token:
        kq = st.hist_k[i, :, :nb].cpu().numpy().astype(np.float32)      # [H, nb, 64, D]
        vq = st.hist_v[i, :, :nb].cpu().numpy().astype(np.float32)
        ksc = st.k_tscale[i, :, :nb * 64].cpu().float().numpy().reshape(8, nb, 64, 1)
        vsc = st.v_tscale[i, :, :nb * 64].cpu().float().numpy().reshape(8, nb, 64, 1)
        ob.hist_k[:nb] = O.bf16_round(kq * ksc).transpose(1, 2, 0, 3)
        ob.hist_v[:nb] = O.bf16_round(vq * vsc).transpose(1, 2, 0, 3)
    return ob


@pytest.mark.parametrize("quant,layout,splits_expected,rel,abs_tol", [
    (False, "channel_block", 0, 2.0 ** -7, 2e-5),
    (True, "channel_block", 0, 2.0 ** -6, 2e-4),
    (True, "token", 0, 2.0 ** -6, 2e-4),
])
def test_headline_36_layer_32k_step_matches_oracle(quant, layout, splits_expected, rel, abs_tol):
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime

    dev = torch.device("cuda:0")
    cfg = M12Config(max_model_len=T, top_k_blocks=32, quant_history=quant, quant_scale_layout=layout)
    model = M12ModelRuntime(L, cfg, device=dev)
    kh = torch.empty(L, T, 8, 128, dtype=torch.bfloat16, device=dev)
    vh = torch.empty_like(kh)
    for i in range(L):
        k, v, _, _ = workload.history(T, SEED + i, device=dev)
        kh[i].copy_(k)
        vh[i].copy_(v)
    model.prefill(kh, vh)
    nb = model.nblocks_filled
    assert nb == 512
    oracles = {i: _oracle_for_layer(model, i, kh, vh, quant, layout) for i in SAMPLED}
    del kh, vh
    n = model.core.effective_k(32)
    assert model.core.decode_splits(n) == splits_expected
    qs, ks, vs = workload.decode_inputs(STEPS, SEED, device=dev, layers=L)
    worst = 0.0
    for s in range(STEPS):
        out = model.decode(qs[s], ks[s], vs[s])
        ids = model.last_ids_dev[:, 0, :model.last_n_selected].cpu()
        for i, ob in oracles.items():
            ids_or, _, o_ref = ob.decode(to_np(qs[s, i]), to_np(ks[s, i]), to_np(vs[s, i]))
            assert ids[i].tolist() == ids_or.tolist(), f"step {s} layer {i}: ids differ"
            worst = max(worst, assert_close_bf16(to_np(out[i]), o_ref, rel=rel, abs_tol=abs_tol))
    print(f"[headline 36L x 32K {('int8 ' + layout) if quant else 'bf16'}, splits {splits_expected}] "
          f"max |err| {worst:.3e}", flush=True)


TV, TQ = 16384, 6


@pytest.mark.parametrize("quant,layout,rel,abs_tol", [
    (False, "channel_block", 2.0 ** -7, 2e-5),
    (True, "channel_block", 2.0 ** -6, 2e-4),
    (True, "token", 2.0 ** -6, 2e-4),
])
def test_verify_36_layer_16k_round_matches_oracle(quant, layout, rel, abs_tol):
    """The launch the verify benchmark times: M12ModelRuntime.verify(lossless)
    over 36 layers of 16384-token histories, 6 draft tokens, the automatic
    kernel choice (the wide few-query kernel in its tiered plan: 3 splits
    for the first 170 of the 288 (layer, KV head) groups, 4 for the rest),
    the benchmark's
    histories (same seeds) and draft tokens of its shapes.  On four sampled
    layers the union of the per-query selections must
    equal the oracle's and the outputs must match the fp64 oracle
    (m12_runtime.py:656-758, :1057-1087); then a commit and a decode step."""
    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime

    dev = torch.device("cuda:0")
    cfg = M12Config(max_model_len=TV + 64, top_k_blocks=32, quant_history=quant,
                    quant_scale_layout=layout)
    model = M12ModelRuntime(L, cfg, device=dev)
    kh = torch.empty(L, TV, 8, 128, dtype=torch.bfloat16, device=dev)
    vh = torch.empty_like(kh)
    for i in range(L):
        k, v, _, _ = workload.history(TV, SEED + i, device=dev)
        kh[i].copy_(k)
        vh[i].copy_(v)
    model.prefill(kh, vh)
    nb = model.nblocks_filled
    assert nb == 256
    oracles = {i: _oracle_for_layer(model, i, kh, vh, quant, layout) for i in SAMPLED}
    del kh, vh
    g = torch.Generator(device=dev).manual_seed(SEED + 31)
    q = torch.randn(L, TQ, 32, 128, generator=g, device=dev).to(torch.bfloat16)
    k = (torch.randn(L, TQ, 8, 128, generator=g, device=dev) * 128 ** -0.5).to(torch.bfloat16)
    v = (torch.randn(L, TQ, 8, 128, generator=g, device=dev) * 128 ** -0.5).to(torch.bfloat16)
    out = model.verify(q, k, v, lossless=True)
    union = model.last_union_dev.cpu()
    count = model.last_union_count_dev.cpu()
    worst = 0.0
    for i, ob in oracles.items():
        ids_or, o_ref = ob.verify_tokens(to_np(q[i]), to_np(k[i]), to_np(v[i]), lossless=True)
        assert union[i, :int(count[i])].tolist() == ids_or.tolist(), f"layer {i}: union differs"
        worst = max(worst, assert_close_bf16(to_np(out[i]), o_ref, rel=rel, abs_tol=abs_tol))
    # accept 4 of the 6 tokens, then one decode step sees them in its window
    model.commit_verified(4)
    qs, ks, vs = workload.decode_inputs(1, SEED, device=dev, layers=L)
    out = model.decode(qs[0], ks[0], vs[0])
    ids = model.last_ids_dev[:, 0, :model.last_n_selected].cpu()
    for i, ob in oracles.items():
        ob.commit_verified(4)
        ids_or, _, o_ref = ob.decode(to_np(qs[0, i]), to_np(ks[0, i]), to_np(vs[0, i]))
        assert ids[i].tolist() == ids_or.tolist(), f"decode after verify, layer {i}: ids differ"
        worst = max(worst, assert_close_bf16(to_np(out[i]), o_ref, rel=rel, abs_tol=abs_tol))
    print(f"[verify 36L x 16K {('int8 ' + layout) if quant else 'bf16'}] max |err| {worst:.3e}", flush=True)
