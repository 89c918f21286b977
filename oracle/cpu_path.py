"""CPU restatement of the reference's decode layer-step op sequence (for the tests and the CPU-baseline timing only).

Used by bench.py's ``cpu_baseline`` leg to time the reference's algorithm on
the host cores of the GPU box; never part of the shipped path.  It performs
the same torch-CPU operations, in the same order, as the reference's
``M12LayerRuntime.decode`` with the history in host memory:

1. recent window shift-left + append            m12_runtime.py:1164-1172
2. fp32 einsum "nhgd,hbrd->nhgbr" + amax chain  m12_runtime.py:999-1003
3. protected blocks -> -inf, topk(k)            m12_runtime.py:1009-1014, :1033
4. token-index index_select gather of K and V   m12_runtime.py:1222-1230
5. pack [selected | sink | recent]              m12_runtime.py:1280-1308
6. fp32 einsum attention + softmax -> bf16      m12_runtime.py:867-873
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


class CpuLayer:
    """One layer's host-side state in the reference's token-major layout."""

    def __init__(self, hist_k, hist_v, reps, sink_k, sink_v, recent_k, recent_v,
                 protected, top_k=32, scale=128.0 ** -0.5, block_size=64):
        self.flat_k = hist_k.reshape(-1, hist_k.shape[-2], hist_k.shape[-1]).contiguous()
        self.flat_v = hist_v.reshape(-1, hist_v.shape[-2], hist_v.shape[-1]).contiguous()
        self.reps = reps.contiguous()                  # [Hkv, nb, r, D] bf16
        self.nblocks = reps.shape[1]
        self.sink_k, self.sink_v = sink_k.contiguous(), sink_v.contiguous()   # [S, Hkv, D]
        self.recent_k, self.recent_v = recent_k.clone(), recent_v.clone()     # [R, Hkv, D]
        self.prot = torch.tensor(sorted(p for p in protected if p < self.nblocks), dtype=torch.long)
        self.top_k = top_k
        self.scale = scale
        self.B = block_size
        sel = top_k * block_size
        self.stage_k = torch.empty(sel, *self.flat_k.shape[1:], dtype=self.flat_k.dtype)
        self.stage_v = torch.empty_like(self.stage_k)
        total = sel + self.sink_k.shape[0] + self.recent_k.shape[0]
        self.packed_k = torch.empty(total, *self.flat_k.shape[1:], dtype=self.flat_k.dtype)
        self.packed_v = torch.empty_like(self.packed_k)

    def decode(self, q, k, v):
        """q [1, Hq, D], k/v [1, Hkv, D] bf16 -> (ids, o [1, Hq, D] bf16)."""
        B = self.B
        self.recent_k[:-1].copy_(self.recent_k[1:].clone())
        self.recent_v[:-1].copy_(self.recent_v[1:].clone())
        self.recent_k[-1].copy_(k[0])
        self.recent_v[-1].copy_(v[0])

        hkv, d = self.reps.shape[0], self.reps.shape[-1]
        hq = q.shape[1]
        q_g = q.view(1, hkv, hq // hkv, d)
        scores = torch.einsum("nhgd,hbrd->nhgbr", q_g.float(), self.reps.float())
        scores = scores.amax(dim=-1).amax(dim=2).amax(dim=0)
        global_scores = scores.amax(dim=0)
        if self.prot.numel():
            global_scores[self.prot] = float("-inf")
        k_eff = min(self.top_k, max(1, self.nblocks - self.prot.numel()))
        ids = global_scores.topk(k_eff).indices

        sel = k_eff * B
        tok_idx = (ids.view(-1, 1) * B + torch.arange(B, dtype=torch.long)).reshape(-1)
        torch.index_select(self.flat_k, 0, tok_idx, out=self.stage_k[:sel])
        torch.index_select(self.flat_v, 0, tok_idx, out=self.stage_v[:sel])

        s_len, r_len = self.sink_k.shape[0], self.recent_k.shape[0]
        pk, pv = self.packed_k, self.packed_v
        pk[:sel].copy_(self.stage_k[:sel])
        pv[:sel].copy_(self.stage_v[:sel])
        pk[sel:sel + s_len].copy_(self.sink_k)
        pv[sel:sel + s_len].copy_(self.sink_v)
        pk[sel + s_len:sel + s_len + r_len].copy_(self.recent_k)
        pv[sel + s_len:sel + s_len + r_len].copy_(self.recent_v)
        total = sel + s_len + r_len

        qf = q.float().view(1, hkv, hq // hkv, d)
        kf, vf = pk[:total].float(), pv[:total].float()
        att = torch.einsum("thgd,shd->thgs", qf, kf) * self.scale
        att = F.softmax(att, dim=-1)
        out = torch.einsum("thgs,shd->thgd", att, vf)
        return ids, out.reshape(1, hq, d).to(q.dtype)


def gather_anchor(flat_k, flat_v, id_groups, threads=(1, 2, 4, 8), seconds_each=0.3, block_size=64):
    """The reference's CPU gather microbenchmark (benchmarks/benchmark_m20_gather.py:88-99,
    its "flat token-index" method): for each group of selected block ids,
    token indices id * 64 + arange(64) gather K and V from the pageable
    history [nb * 64, Hkv, D] into pinned staging with index_select -- 8 MiB
    per group at 32 blocks, bf16 [*, 8, 128].  Returns {threads: median us
    per gather}, cycling through the groups, ~seconds_each per thread count.
    """
    import time

    n_tok = id_groups[0].numel() * block_size
    pin = torch.cuda.is_available()
    stage_k = torch.empty(n_tok, *flat_k.shape[1:], dtype=flat_k.dtype, pin_memory=pin)
    stage_v = torch.empty_like(stage_k, pin_memory=pin)
    ar = torch.arange(block_size, dtype=torch.long)
    tok = [(ids.view(-1, 1) * block_size + ar).reshape(-1) for ids in id_groups]
    saved = torch.get_num_threads()
    out = {}
    try:
        for n in threads:
            torch.set_num_threads(n)
            times, i = [], 0
            t_end = time.perf_counter() + seconds_each
            while time.perf_counter() < t_end or len(times) < 5:
                idx = tok[i % len(tok)]
                t0 = time.perf_counter()
                torch.index_select(flat_k, 0, idx, out=stage_k)
                torch.index_select(flat_v, 0, idx, out=stage_v)
                times.append(time.perf_counter() - t0)
                i += 1
            times.sort()
            out[n] = times[len(times) // 2] * 1e6
    finally:
        torch.set_num_threads(saved)
    return out
