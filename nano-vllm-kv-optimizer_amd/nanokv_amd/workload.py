"""Seeded synthetic Qwen3-4B-shaped attention inputs for the sparse layer-step.

Attention shape: 32 query heads, 8 KV heads, head_dim 128 (GQA 4:1), 64-token
blocks.  History K/V ~ N(0, 1)/sqrt(128) and queries ~ N(0, 1), drawn in fp32
and rounded to bf16; layer L of a run uses its own generator seeded with
``seed + L``.  Three non-protected blocks are planted so that selection has a
clear winner set: for every token t of a planted block and KV head h,
``k[t, h] += 0.5 * q[4h] / |q[4h]|`` (the first query head of the group).
"""

from __future__ import annotations

import torch

NUM_HEADS = 32
NUM_KV_HEADS = 8
HEAD_DIM = 128
BLOCK = 64


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def history(num_tokens: int, seed: int, *, device="cpu", num_planted: int = 3,
            recent_tokens: int = 512):
    """(k, v, q, planted) for one layer.

    k, v: [T, Hkv, D] bf16; q: [Hq, D] bf16 (the decode query the planted
    blocks are aligned with); planted: sorted list of block ids in
    [1, nblocks - recent_tokens/64 - 1).
    """
    g = _gen(seed, device)
    scale = HEAD_DIM ** -0.5
    k = torch.randn(num_tokens, NUM_KV_HEADS, HEAD_DIM, generator=g, device=device) * scale
    v = torch.randn(num_tokens, NUM_KV_HEADS, HEAD_DIM, generator=g, device=device) * scale
    q = torch.randn(NUM_HEADS, HEAD_DIM, generator=g, device=device)
    nb = (num_tokens + BLOCK - 1) // BLOCK
    lo, hi = 1, nb - recent_tokens // BLOCK - 1
    planted: list[int] = []
    if num_planted and hi - lo >= num_planted:
        perm = torch.randperm(hi - lo, generator=g, device=device)[:num_planted] + lo
        planted = sorted(int(b) for b in perm.tolist())
        qb = q.to(torch.bfloat16).float()
        for b in planted:
            t0, t1 = b * BLOCK, min(num_tokens, (b + 1) * BLOCK)
            for h in range(NUM_KV_HEADS):
                qh = qb[4 * h]
                k[t0:t1, h] += 0.5 * qh / qh.norm()
    return k.to(torch.bfloat16), v.to(torch.bfloat16), q.to(torch.bfloat16), planted


def decode_inputs(steps: int, seed: int, *, device="cpu", layers: int = 1):
    """Per-step decode inputs: q [steps, L, 1, Hq, D], k/v [steps, L, 1, Hkv, D] bf16."""
    g = _gen(seed + 7919, device)
    scale = HEAD_DIM ** -0.5
    q = torch.randn(steps, layers, 1, NUM_HEADS, HEAD_DIM, generator=g, device=device)
    k = torch.randn(steps, layers, 1, NUM_KV_HEADS, HEAD_DIM, generator=g, device=device) * scale
    v = torch.randn(steps, layers, 1, NUM_KV_HEADS, HEAD_DIM, generator=g, device=device) * scale
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def prefill_chunk_inputs(num_tokens: int, seed: int, *, device="cpu", layers: int = 1):
    """A later prefill chunk: q [L, T, Hq, D] ~ N(0,1), k/v [L, T, Hkv, D] ~ N(0,1)/sqrt(D), bf16."""
    g = _gen(seed + 104729, device)
    scale = HEAD_DIM ** -0.5
    q = torch.randn(layers, num_tokens, NUM_HEADS, HEAD_DIM, generator=g, device=device)
    k = torch.randn(layers, num_tokens, NUM_KV_HEADS, HEAD_DIM, generator=g, device=device) * scale
    v = torch.randn(layers, num_tokens, NUM_KV_HEADS, HEAD_DIM, generator=g, device=device) * scale
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
