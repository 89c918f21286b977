"""Write the golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Inputs are the seeded synthetic workloads of nanokv_amd.workload (CPU
generator, so they regenerate bit-identically); the fixtures keep only their
sha256 digests plus the oracle's outputs:

* c1_decode_8k.npz   8192-token bf16 history, one decode step with the
                     planted query: representative picks, selected ids and
                     scores (+ the gap at the Top-32 cutoff), fp64 output.
* c3_int8_8k.npz     the same history stored int8 (K per-channel, V
                     per-block scales): scales, ids, output.
* c5_verify_4k.npz   4096-token history, 6 verify queries, lossless
                     (per-query Top-32 + union + allowed mask) and shared
                     selection: union, allowed, ids, outputs.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "nano-vllm-kv-optimizer_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

from nanokv_amd import workload  # noqa: E402
from oracle import nkv_oracle as O  # noqa: E402


def sha(t) -> str:
    return hashlib.sha256(t.contiguous().view(-1).view(__import__("torch").int16).numpy().tobytes()).hexdigest()


def f32(t):
    return t.float().numpy()


def inputs(T, seed, steps=1):
    k, v, q, planted = workload.history(T, seed)
    qs, ks, vs = workload.decode_inputs(steps, seed)
    return k, v, q, planted, qs, ks, vs


def digests(k, v, q, qs, ks, vs):
    return np.array([sha(k), sha(v), sha(q), sha(qs), sha(ks), sha(vs)])


def cutoff_gap(scores, protected, k):
    s = np.array(scores, np.float32, copy=True)
    prot = [p for p in protected if 0 <= p < s.shape[0]]
    s[prot] = -np.inf
    srt = np.sort(s)[::-1]
    return float(srt[k - 1] - srt[k]) if s.shape[0] > k else float("inf")


def make_c1():
    T, seed = 8192, 1234
    k, v, q, planted, qs, ks, vs = inputs(T, seed)
    ob = O.M12Oracle(O.OracleConfig())
    ob.store_kv(f32(k), f32(v))
    nb = ob.nblocks_filled
    sel, _, margins = O.build_reps(f32(k).reshape(nb, 64, 8, 128), 4)
    q1 = f32(q)[None]
    scores = O.block_scores(q1, ob.reps, nb, 8)
    ids, vals, o = ob.decode(q1, f32(ks[0, 0]), f32(vs[0, 0]))
    np.savez_compressed(
        os.path.join(HERE, "c1_decode_8k.npz"), T=T, seed=seed, planted=np.array(planted),
        digests=digests(k, v, q, qs, ks, vs), rep_sel=sel.astype(np.int16),
        rep_margin_min=float(margins.min()), scores=scores, ids=ids, vals=vals,
        gap=cutoff_gap(scores, ob.protected_blocks, 32), out=o.astype(np.float32))
    print(f"c1: ids {ids[:6].tolist()}... planted {planted} gap {cutoff_gap(scores, ob.protected_blocks, 32):.3e}")


def make_c3():
    T, seed = 8192, 4321
    k, v, q, planted, qs, ks, vs = inputs(T, seed)
    ob = O.M12Oracle(O.OracleConfig(quant_history=True))
    ob.store_kv(f32(k), f32(v))
    nb = ob.nblocks_filled
    ids, vals, o = ob.decode(f32(q)[None], f32(ks[0, 0]), f32(vs[0, 0]))
    hk = hashlib.sha256(ob.hist_kq[:nb].tobytes()).hexdigest()
    hv = hashlib.sha256(ob.hist_vq[:nb].tobytes()).hexdigest()
    np.savez_compressed(
        os.path.join(HERE, "c3_int8_8k.npz"), T=T, seed=seed, planted=np.array(planted),
        digests=digests(k, v, q, qs, ks, vs), k_scale=ob.k_scale, v_scale=ob.v_scale[:nb],
        kq_sha=hk, vq_sha=hv, ids=ids, vals=vals, out=o.astype(np.float32))
    print(f"c3: ids {ids[:6].tolist()}... planted {planted}")


def make_c5():
    T, seed, tq = 4096, 555, 6
    k, v, q, planted, qs, ks, vs = inputs(T, seed, steps=tq)
    qv = f32(qs[:, 0, 0])          # [6, 32, 128]
    kv_ = f32(ks[:, 0, 0])         # [6, 8, 128]
    vv = f32(vs[:, 0, 0])
    out = {}
    for lossless in (True, False):
        ob = O.M12Oracle(O.OracleConfig())
        ob.store_kv(f32(k), f32(v))
        if lossless:
            union, allowed, tops = O.select_per_query(qv, ob.reps, ob.nblocks_filled, 8,
                                                      ob.protected_blocks, 32)
            out["union"], out["allowed"], out["tops"] = union, allowed, tops
        ids, o = ob.verify_tokens(qv, kv_, vv, lossless=lossless)
        key = "lossless" if lossless else "shared"
        out[f"ids_{key}"] = ids
        out[f"out_{key}"] = o.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "c5_verify_4k.npz"), T=T, seed=seed, tq=tq,
                        digests=digests(k, v, q, qs, ks, vs), **out)
    print(f"c5: union {len(out['union'])} blocks, shared ids {out['ids_shared'][:6].tolist()}...")


if __name__ == "__main__":
    make_c1()
    make_c3()
    make_c5()
