"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the regenerated inputs still hash to the recorded digests and the oracle
reproduces the recorded outputs exactly.  GPU: the HIP path reproduces the
recorded representatives, selected ids (exact) and outputs (~1 bf16 ulp)."""

import os

import numpy as np
import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import assert_close_bf16, to_np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def _inputs(fx, steps=1):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    k, v, q, planted, qs, ks, vs = mg.inputs(int(fx["T"]), int(fx["seed"]), steps)
    assert mg.digests(k, v, q, qs, ks, vs).tolist() == fx["digests"].tolist(), "input generator drifted"
    return k, v, q, planted, qs, ks, vs


def test_c1_oracle_reproduces_fixture():
    fx = _load("c1_decode_8k.npz")
    k, v, q, planted, qs, ks, vs = _inputs(fx)
    assert planted == fx["planted"].tolist()
    ob = O.M12Oracle(O.OracleConfig())
    ob.store_kv(to_np(k), to_np(v))
    ids, vals, o = ob.decode(to_np(q)[None], to_np(ks[0, 0]), to_np(vs[0, 0]))
    assert ids.tolist() == fx["ids"].tolist()
    assert np.array_equal(vals, fx["vals"])
    assert np.array_equal(o.astype(np.float32), fx["out"])
    assert set(fx["planted"].tolist()) <= set(ids[:3].tolist())
    assert float(fx["gap"]) > 1e-4          # cutoff well above fp32 accumulation error


def test_c3_oracle_reproduces_fixture():
    fx = _load("c3_int8_8k.npz")
    k, v, q, planted, qs, ks, vs = _inputs(fx)
    ob = O.M12Oracle(O.OracleConfig(quant_history=True))
    ob.store_kv(to_np(k), to_np(v))
    ids, vals, o = ob.decode(to_np(q)[None], to_np(ks[0, 0]), to_np(vs[0, 0]))
    assert np.array_equal(ob.k_scale, fx["k_scale"])
    assert ids.tolist() == fx["ids"].tolist()
    assert np.array_equal(o.astype(np.float32), fx["out"])


def test_c5_oracle_reproduces_fixture():
    fx = _load("c5_verify_4k.npz")
    tq = int(fx["tq"])
    k, v, q, planted, qs, ks, vs = _inputs(fx, tq)
    for lossless in (True, False):
        ob = O.M12Oracle(O.OracleConfig())
        ob.store_kv(to_np(k), to_np(v))
        ids, o = ob.verify_tokens(to_np(qs[:, 0, 0]), to_np(ks[:, 0, 0]), to_np(vs[:, 0, 0]),
                                  lossless=lossless)
        key = "lossless" if lossless else "shared"
        assert ids.tolist() == fx[f"ids_{key}"].tolist()
        assert np.array_equal(o.astype(np.float32), fx[f"out_{key}"])


@pytest.mark.gpu
def test_c1_gpu_matches_fixture():
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    fx = _load("c1_decode_8k.npz")
    k, v, q, planted, qs, ks, vs = _inputs(fx)
    rt = M12LayerRuntime(0, M12Config(max_model_len=int(fx["T"])))
    rt.prefill_first(None, k.cuda(), v.cuda())
    # GPU representatives pick the same tokens as the fixture
    nb = rt.nblocks_filled
    reps = rt.reps_gpu[:, :nb].cpu()
    kb = k.view(nb, 64, 8, 128)
    sel = fx["rep_sel"].astype(np.int64)
    want = torch.stack([kb[torch.arange(nb)[:, None], torch.from_numpy(sel[:, :, j]), torch.arange(8)[None, :]]
                        for j in range(4)], dim=2)               # [nb, 8, 4, 128]
    assert torch.equal(reps, want.permute(1, 0, 2, 3)), "representative picks differ from the fixture"
    out = rt.decode(q.unsqueeze(0).cuda(), ks[0, 0].cuda(), vs[0, 0].cuda())
    assert rt.last_block_ids.tolist() == fx["ids"].tolist()
    assert_close_bf16(to_np(out), fx["out"].astype(np.float64))


@pytest.mark.gpu
def test_c3_gpu_matches_fixture():
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    fx = _load("c3_int8_8k.npz")
    k, v, q, planted, qs, ks, vs = _inputs(fx)
    rt = M12LayerRuntime(0, M12Config(max_model_len=int(fx["T"]), quant_history=True))
    rt.prefill_first(None, k.cuda(), v.cuda())
    assert np.array_equal(rt.store.k_scale[0].cpu().numpy(), fx["k_scale"])
    out = rt.decode(q.unsqueeze(0).cuda(), ks[0, 0].cuda(), vs[0, 0].cuda())
    assert rt.last_block_ids.tolist() == fx["ids"].tolist()
    assert_close_bf16(to_np(out), fx["out"].astype(np.float64), rel=2.0 ** -6, abs_tol=2e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("lossless", [True, False])
def test_c5_gpu_verify_matches_fixture(lossless):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    fx = _load("c5_verify_4k.npz")
    tq = int(fx["tq"])
    k, v, q, planted, qs, ks, vs = _inputs(fx, tq)
    rt = M12LayerRuntime(0, M12Config(max_model_len=int(fx["T"]) + 64))
    rt.prefill_first(None, k.cuda(), v.cuda())
    rt.verify_lossless = lossless
    out = rt.verify_tokens(qs[:, 0, 0].cuda(), ks[:, 0, 0].cuda(), vs[:, 0, 0].cuda())
    key = "lossless" if lossless else "shared"
    assert rt.last_verify_block_ids.tolist() == fx[f"ids_{key}"].tolist()
    assert_close_bf16(to_np(out), fx[f"out_{key}"].astype(np.float64))
