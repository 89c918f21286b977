"""Device-ring decode (nkv_decode_step_ring) and its HIP-graph replay.

Once the sink and recent window are full, the only decode argument that
changes from step to step is the ring position (m12_runtime.py:1164-1172's
shift + append).  nkv_decode_step_ring keeps it in device memory and advances
it on the device, so one decode step can be captured and replayed.

Checks, on the same inputs:
* a runtime with device_ring set is bit-identical to the regular path (output
  and selected ids) for 600 steps, through the wrap of the 512-slot ring, and
  its device ring value ends equal to the host's;
* a captured decode step, replayed 520 times with the regular runtime's eager
  steps and a synchronisation between replays, matches it bit for bit on
  every replay;
* a host-side ring move (reset + new prefill) is picked up by the next
  device-ring step.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _pair(T=1024, seed=5):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime

    cfg = M12Config(max_model_len=4096, top_k_blocks=8)
    a, b = M12LayerRuntime(0, cfg), M12LayerRuntime(0, cfg)
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = (torch.randn(T, HKV, D, generator=g, device="cuda") * D ** -0.5).bfloat16()
    v = torch.randn(T, HKV, D, generator=g, device="cuda").bfloat16()
    for rt in (a, b):
        rt.prefill_first(None, k, v)
    b.device_ring = True
    return a, b


def _steps(n, seed=9):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(n, 1, HQ, D, generator=g, device="cuda").bfloat16(),
            (torch.randn(n, 1, HKV, D, generator=g, device="cuda") * D ** -0.5).bfloat16(),
            torch.randn(n, 1, HKV, D, generator=g, device="cuda").bfloat16())


def test_device_ring_matches_regular_decode_through_the_ring_wrap():
    a, b = _pair()
    assert b.device_ring_ready() and a.valid_len == 1024
    qs, ks, vs = _steps(600)
    for i in range(600):
        oa = a.decode(qs[i], ks[i], vs[i])
        ob = b.decode(qs[i], ks[i], vs[i])
        assert torch.equal(oa, ob), f"step {i}"
        assert torch.equal(a.last_block_ids, b.last_block_ids), f"step {i}"
    c = b._core
    assert c.ring_start == a._core.ring_start and c.valid_len == a.valid_len == 1624
    assert c._ring_dev.tolist() == [c.ring_start]


def test_captured_decode_step_replays_match_eager_decode():
    a, b = _pair(seed=6)
    qs, ks, vs = _steps(522, seed=10)
    q_s, k_s, v_s = qs[0].clone(), ks[0].clone(), vs[0].clone()
    # warm-up step (allocates the device ring and workspaces), on both runtimes
    assert torch.equal(a.decode(qs[0], ks[0], vs[0]), b.decode(q_s, k_s, v_s))
    state = b.decode_state()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = b.decode(q_s, k_s, v_s)
    b.restore_decode_state(state)
    assert b.decode_state() == state
    for i in range(1, 522):
        q_s.copy_(qs[i])
        k_s.copy_(ks[i])
        v_s.copy_(vs[i])
        graph.replay()
        b.ring_replayed()
        oa = a.decode(qs[i], ks[i], vs[i])     # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, oa), f"replay {i}"
        assert torch.equal(b.last_block_ids, a.last_block_ids), f"replay {i}"
    assert b._core._ring_dev.tolist() == [b._core.ring_start] == [a._core.ring_start]


def test_host_ring_move_is_picked_up_by_the_next_device_ring_step():
    a, b = _pair(seed=7)
    qs, ks, vs = _steps(3, seed=11)
    for i in range(3):
        assert torch.equal(a.decode(qs[i], ks[i], vs[i]), b.decode(qs[i], ks[i], vs[i]))
    # a new sequence of a different length: the ring start changes on the host
    g = torch.Generator(device="cuda").manual_seed(8)
    k = (torch.randn(700, HKV, D, generator=g, device="cuda") * D ** -0.5).bfloat16()
    v = torch.randn(700, HKV, D, generator=g, device="cuda").bfloat16()
    for rt in (a, b):
        rt.reset()
        rt.prefill_first(None, k, v)
    qs, ks, vs = _steps(4, seed=12)
    for i in range(4):
        assert torch.equal(a.decode(qs[i], ks[i], vs[i]), b.decode(qs[i], ks[i], vs[i])), f"step {i}"
    assert b._core._ring_dev.tolist() == [b._core.ring_start] == [a._core.ring_start]
