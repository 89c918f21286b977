"""Seeded sweeps of decode, chunked-prefill and verify configurations against the oracle.

Beyond the Qwen3-4B attention shape of the other decode tests: GQA ratios
1-16, r = 1, 2, 4, 8 representatives, budgets 1-200 (including more than the
history offers, and more than one wavefront's 64 lanes), explicit attention
split counts (a multiple of 4, and more splits than segments, so some
workgroups attend nothing), ragged histories, bf16 and int8 history.

Per decode step: selected ids bit-exact against the oracle, outputs within
the bf16 bar (tests/_util.assert_close_bf16).  The representatives are the
GPU's (the rep builder is pinned on its own), so each case checks the
layer-step itself.
"""

import pytest
import torch

from oracle import nkv_oracle as O
from tests._util import assert_close_bf16, to_np

pytestmark = pytest.mark.gpu

D = 128

# (Hq, Hkv, r, T, top_k, attend_splits, int8, seed)
CASES = [
    (16, 16, 4, 3000, 16, 3, False, 1),     # G = 1
    (32, 16, 2, 5000, 32, 5, False, 2),     # G = 2, r = 2
    (64, 8, 8, 2500, 8, 2, False, 3),       # G = 8, r = 8
    (64, 4, 1, 4100, 64, 7, False, 4),      # G = 16, r = 1, a full wavefront of ids
    (32, 8, 4, 700, 1, 1, False, 5),        # top-1, one split
    (32, 8, 4, 300, 32, 8, False, 6),       # short history, more splits than segments
    (32, 8, 4, 9000, 48, 4, False, 7),      # an explicit multiple of 4
    (32, 4, 4, 6000, 20, None, True, 8),    # int8, G = 8
    (16, 8, 2, 2049, 32, 6, True, 9),       # int8, ragged last block
    (32, 8, 4, 20000, 128, None, False, 10),  # k > 64: the sorting-network path
    (8, 8, 4, 1500, 12, 2, False, 11),      # Hq = Hkv = 8
    (32, 8, 4, 64 * 40, 200, None, False, 12),  # budget above the 31 selectable blocks
]


@pytest.mark.parametrize("hq,hkv,r,T,top_k,splits,int8,seed", CASES)
def test_decode_sweep_against_oracle(hq, hkv, r, T, top_k, splits, int8, seed):
    from nanokv_amd.sparse import M12Config, M12LayerRuntime

    print(f"case Hq={hq} Hkv={hkv} r={r} T={T} k={top_k} splits={splits} int8={int8}", flush=True)
    cfg = M12Config(max_model_len=T + 64, num_heads=hq, num_kv_heads=hkv, r=r, top_k_blocks=top_k,
                    attend_splits=splits, quant_history=int8)
    rt = M12LayerRuntime(0, cfg)
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    v = (torch.randn(T, hkv, D, generator=g) * D ** -0.5).bfloat16()
    rt.prefill_first(None, k.cuda(), v.cuda())

    ob = O.M12Oracle(O.OracleConfig(num_heads=hq, num_kv_heads=hkv, r=r, top_k_blocks=top_k,
                                    quant_history=int8))
    ob.store_kv(to_np(k), to_np(v), with_reps=False)
    nb = rt.nblocks_filled
    assert nb == ob.nblocks_filled
    ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])

    for step in range(2):
        q = torch.randn(1, hq, D, generator=g).bfloat16()
        kn = (torch.randn(1, hkv, D, generator=g) * D ** -0.5).bfloat16()
        vn = (torch.randn(1, hkv, D, generator=g) * D ** -0.5).bfloat16()
        out = rt.decode(q.cuda(), kn.cuda(), vn.cuda())
        ids_or, _, o_ref = ob.decode(to_np(q), to_np(kn), to_np(vn))
        assert rt.last_block_ids.tolist() == ids_or.tolist(), f"step {step}: ids differ"
        assert_close_bf16(to_np(out), o_ref)
        assert rt.valid_len == ob.valid_len


# (Hq, Hkv, r, history T, chunk lengths, top_k, int8, seed)
PREFILL_CASES = [
    (16, 16, 4, 1800, (40, 300), 16, False, 21),     # G = 1: 128 tokens per query tile
    (64, 4, 2, 2500, (17, 130), 32, False, 22),      # G = 16: 8 tokens per query tile
    (32, 16, 8, 3100, (9, 257), 12, True, 23),       # G = 2, r = 8, int8
    (8, 8, 1, 900, (2, 64, 65), 8, False, 24),       # two-token chunk, block-aligned and ragged
]


@pytest.mark.parametrize("hq,hkv,r,T,chunks,top_k,int8,seed", PREFILL_CASES)
def test_prefill_sweep_against_oracle(hq, hkv, r, T, chunks, top_k, int8, seed):
    """Later prefill chunks (query summaries, selection, [selected | sink |
    previous recent | causal chunk]) on both attention kernels (few-query
    kernel for short chunks, matrix cores for long ones) against the oracle:
    ids bit-exact, outputs within the bf16-probability bar of the prefill
    tests."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    from tests._util import PREFILL_TOL

    print(f"case Hq={hq} Hkv={hkv} r={r} T={T} chunks={chunks} k={top_k} int8={int8}", flush=True)
    blocks = -(-T // 64) + sum(-(-n // 64) for n in chunks)   # every stored chunk starts a block
    cfg = M12Config(max_model_len=64 * blocks, num_heads=hq, num_kv_heads=hkv, r=r,
                    top_k_blocks=top_k, quant_history=int8)
    rt = M12LayerRuntime(0, cfg)
    ob = O.M12Oracle(O.OracleConfig(num_heads=hq, num_kv_heads=hkv, r=r, top_k_blocks=top_k,
                                    quant_history=int8))
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(T, hkv, D, generator=g) * 0.09).bfloat16()
    v = (torch.randn(T, hkv, D, generator=g) * 0.09).bfloat16()
    rt.prefill_first(None, k.cuda(), v.cuda())
    ob.store_kv(to_np(k), to_np(v), with_reps=False)
    for i, n in enumerate(chunks):
        nb = rt.nblocks_filled
        ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])
        q = torch.randn(n, hq, D, generator=g).bfloat16()
        kc = (torch.randn(n, hkv, D, generator=g) * 0.09).bfloat16()
        vc = (torch.randn(n, hkv, D, generator=g) * 0.09).bfloat16()
        out = rt.prefill_chunk(q.cuda(), kc.cuda(), vc.cuda())
        ids_or, o_ref = ob.prefill_chunk(to_np(q), to_np(kc), to_np(vc))
        assert rt.last_prefill_block_ids.tolist() == ids_or.tolist(), f"chunk {i}: ids differ"
        assert_close_bf16(to_np(out), o_ref, **PREFILL_TOL)


# (Hq, Hkv, r, history T, draft tokens, top_k, lossless, seed)
VERIFY_CASES = [
    (16, 16, 4, 5000, 2, 16, False, 31),   # G = 1, 2 queries
    (64, 4, 2, 6000, 8, 32, True, 32),     # G = 16: 8 queries = 128 rows, matrix cores, per-query masks
    (32, 16, 8, 4000, 5, 24, True, 33),    # G = 2, r = 8: 10 rows on the few-query kernel
    (32, 4, 4, 5000, 3, 32, True, 34),     # G = 8: 24 rows, the few-query kernel's wide form
    (32, 8, 2, 6000, 7, 20, False, 35),    # G = 4: 28 rows (wide), shared selection
]


@pytest.mark.parametrize("hq,hkv,r,T,tq,top_k,lossless,seed", VERIFY_CASES)
def test_verify_sweep_against_oracle(hq, hkv, r, T, tq, top_k, lossless, seed):
    """Speculative verify (shared or lossless per-query selection), a partial
    commit, then one decode step, against the oracle."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime
    from tests._util import PREFILL_TOL

    print(f"case Hq={hq} Hkv={hkv} r={r} T={T} tq={tq} k={top_k} lossless={lossless}", flush=True)
    cfg = M12Config(max_model_len=T + 64, num_heads=hq, num_kv_heads=hkv, r=r, top_k_blocks=top_k)
    rt = M12LayerRuntime(0, cfg)
    ob = O.M12Oracle(O.OracleConfig(num_heads=hq, num_kv_heads=hkv, r=r, top_k_blocks=top_k))
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(T, hkv, D, generator=g) * 0.09).bfloat16()
    v = (torch.randn(T, hkv, D, generator=g) * 0.09).bfloat16()
    rt.prefill_first(None, k.cuda(), v.cuda())
    ob.store_kv(to_np(k), to_np(v), with_reps=False)
    nb = rt.nblocks_filled
    ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])
    rt.verify_lossless = lossless
    q = torch.randn(tq, hq, D, generator=g).bfloat16()
    kc = (torch.randn(tq, hkv, D, generator=g) * 0.09).bfloat16()
    vc = (torch.randn(tq, hkv, D, generator=g) * 0.09).bfloat16()
    out = rt.verify_tokens(q.cuda(), kc.cuda(), vc.cuda())
    ids_or, o_ref = ob.verify_tokens(to_np(q), to_np(kc), to_np(vc), lossless=lossless)
    assert rt.last_verify_block_ids.tolist() == ids_or.tolist()
    assert_close_bf16(to_np(out), o_ref, **PREFILL_TOL)
    rt.commit_verified(tq - 1)
    ob.commit_verified(tq - 1)
    assert rt.valid_len == ob.valid_len
    q = torch.randn(1, hq, D, generator=g).bfloat16()
    kn = (torch.randn(1, hkv, D, generator=g) * 0.09).bfloat16()
    vn = (torch.randn(1, hkv, D, generator=g) * 0.09).bfloat16()
    out = rt.decode(q.cuda(), kn.cuda(), vn.cuda())
    ids_or, _, o_ref = ob.decode(to_np(q), to_np(kn), to_np(vn))
    assert rt.last_block_ids.tolist() == ids_or.tolist()
    assert_close_bf16(to_np(out), o_ref)


# (Hq, Hkv, history T, draft tokens, lossless, force the few-query kernels,
# seed): verify shapes on the wide few-query kernel (two 16-column MFMA tiles
# per group of up to 32 query rows) beyond the Qwen3-4B shape
WIDE_CASES = [
    (16, 16, 3000, 16, True, False, 51),   # G = 1: 16 rows, one tile (the 16-row kernel)
    (16, 16, 3000, 20, False, False, 52),  # G = 1: 20 rows, one wide group, shared selection
    (32, 16, 3500, 12, True, False, 53),   # G = 2: 24 rows, per-query masks
    (64, 4, 2500, 2, True, False, 54),     # G = 16: 32 rows, a full wide group
    (64, 4, 2500, 3, False, True, 55),     # G = 16: 48 rows, two wide groups (32 + 16), forced
    (32, 32, 2000, 40, False, True, 56),   # G = 1: 40 rows, two wide groups (32 + 8), forced
]


@pytest.mark.parametrize("hq,hkv,T,tq,lossless,force,seed", WIDE_CASES)
def test_verify_wide_kernel_shapes_against_oracle(hq, hkv, T, tq, lossless, force, seed):
    """Verify rounds whose query rows take the wide few-query kernel (or, where
    noted, are forced onto the few-query kernels), against the oracle: ids
    bit-exact, outputs within the bf16 bar (fp32-accurate P.V)."""
    from nanokv_amd.sparse import M12Config, M12LayerRuntime

    print(f"case Hq={hq} Hkv={hkv} T={T} tq={tq} lossless={lossless} force={force}", flush=True)
    top_k = 16
    cfg = M12Config(max_model_len=T + 64, num_heads=hq, num_kv_heads=hkv, top_k_blocks=top_k,
                    mfma_chunk_min_tokens=10000 if force else None)
    rt = M12LayerRuntime(0, cfg)
    ob = O.M12Oracle(O.OracleConfig(num_heads=hq, num_kv_heads=hkv, top_k_blocks=top_k))
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(T, hkv, D, generator=g) * 0.09).bfloat16()
    v = (torch.randn(T, hkv, D, generator=g) * 0.09).bfloat16()
    rt.prefill_first(None, k.cuda(), v.cuda())
    ob.store_kv(to_np(k), to_np(v), with_reps=False)
    nb = rt.nblocks_filled
    ob.reps[:, :nb] = to_np(rt.reps_gpu[:, :nb])
    rt.verify_lossless = lossless
    q = torch.randn(tq, hq, D, generator=g).bfloat16()
    kc = (torch.randn(tq, hkv, D, generator=g) * 0.09).bfloat16()
    vc = (torch.randn(tq, hkv, D, generator=g) * 0.09).bfloat16()
    out = rt.verify_tokens(q.cuda(), kc.cuda(), vc.cuda())
    ids_or, o_ref = ob.verify_tokens(to_np(q), to_np(kc), to_np(vc), lossless=lossless)
    assert rt.last_verify_block_ids.tolist() == ids_or.tolist()
    worst = assert_close_bf16(to_np(out), o_ref)
    print(f"  max |err| {worst:.2e}", flush=True)
