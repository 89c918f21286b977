"""History in pinned host memory (history_tier="host") on the GPU kernels.

The reference keeps its history on the host and gathers + copies the
selected blocks to the GPU every step (m12_runtime.py:185-246, :1212-1311).
The host tier keeps hist_k / hist_v in pinned host memory and the same
kernels read the selected blocks in place through the device mapping
(nkv_host_device_pointer); nothing else changes.  So the bar is bit-identity
with the HBM tier: a host-tier and an HBM-tier runtime driven through the
same sequence (two prefill chunks, decode steps, a lossless verify round
with a partial commit) must produce identical outputs, selections and
stored history in every KV format; the batched model runtime likewise.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).cuda()


def _qkv(t, seed, lead=()):
    return (_rand((*lead, t, HQ, D), seed), _rand((*lead, t, HKV, D), seed + 1, D ** -0.5),
            _rand((*lead, t, HKV, D), seed + 2))


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8_token"])
def test_host_tier_is_bit_identical_to_hbm_tier(fmt):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime

    kw = dict(max_model_len=8192, top_k_blocks=16, quant_history=fmt != "bf16",
              quant_scale_layout="token" if fmt == "int8_token" else "channel_block")
    hbm = M12LayerRuntime(0, M12Config(**kw))
    host = M12LayerRuntime(0, M12Config(history_tier="host", **kw))
    st = host.store
    assert st.history_tier == "host" and not st.hist_k.is_cuda and st.hist_k.is_pinned()
    assert st.hist_v.is_pinned() and st.reps.is_cuda and st.recent_k.is_cuda
    print(f"[host tier {fmt}] prefill", flush=True)
    q, k, v = _qkv(1500, 11)
    for rt in (hbm, host):
        rt.prefill_first(q, k, v)
    q, k, v = _qkv(700, 21)
    assert torch.equal(hbm.prefill_chunk(q, k, v), host.prefill_chunk(q, k, v))
    assert torch.equal(hbm.last_prefill_block_ids, host.last_prefill_block_ids)
    torch.cuda.synchronize()
    nb = hbm.nblocks_filled
    assert torch.equal(hbm.store.hist_k[0, :, :nb].cpu(), st.hist_k[0, :, :nb])
    assert torch.equal(hbm.store.hist_v[0, :, :nb].cpu(), st.hist_v[0, :, :nb])
    print(f"[host tier {fmt}] decode", flush=True)
    for step in range(4):
        q, k, v = _qkv(1, 31 + 3 * step)
        assert torch.equal(hbm.decode(q, k, v), host.decode(q, k, v))
        assert torch.equal(hbm.last_block_ids, host.last_block_ids)
    print(f"[host tier {fmt}] verify", flush=True)
    for rt in (hbm, host):
        rt.verify_mode = True
        rt.verify_lossless = True
    q, k, v = _qkv(6, 51)
    assert torch.equal(hbm.verify_tokens(q, k, v), host.verify_tokens(q, k, v))
    for rt in (hbm, host):
        rt.commit_verified(4)
        rt.verify_mode = False
    q, k, v = _qkv(1, 61)
    assert torch.equal(hbm.decode(q, k, v), host.decode(q, k, v))


def test_model_runtime_host_tier_decode_is_bit_identical():
    from nanokv_amd.sparse import M12Config, M12ModelRuntime

    L = 3
    a = M12ModelRuntime(L, M12Config(max_model_len=8192, top_k_blocks=16))
    b = M12ModelRuntime(L, M12Config(max_model_len=8192, top_k_blocks=16, history_tier="host"))
    _, k, v = _qkv(3000, 71, (L,))
    a.prefill(k, v)
    b.prefill(k, v)
    for step in range(3):
        q, k, v = _qkv(1, 81 + 3 * step, (L,))
        assert torch.equal(a.decode(q, k, v), b.decode(q, k, v))
        assert torch.equal(a.last_ids_dev, b.last_ids_dev)


def test_host_device_pointer_accepts_only_pinned_host_memory():
    from nanokv_amd import _lib

    pinned = torch.zeros(1024, pin_memory=True)
    assert _lib.host_device_pointer(pinned.data_ptr()) != 0
    pageable = torch.zeros(1024)
    with pytest.raises(ValueError, match="host_device_pointer"):
        _lib.host_device_pointer(pageable.data_ptr())
    dev = torch.zeros(1024, device="cuda")
    with pytest.raises(ValueError, match="not pinned host memory"):
        _lib.host_device_pointer(dev.data_ptr())
