"""A Qwen3 decoder whose attention is the sparse layer-step.

The module structure of nanovllm/models/qwen3.py:14-220 (Qwen3Attention,
Qwen3MLP, Qwen3DecoderLayer, Qwen3Model, Qwen3ForCausalLM) on one GPU:

* fused q/k/v and gate/up projections (plain bf16 GEMMs);
* per-head RMSNorm of q and k when the projections carry no bias;
* rotate-half RoPE over the whole head in fp32
  (nanovllm/layers/rotary_embedding.py:6-50), with YaRN scaling when the
  config asks for it (rotary_embedding.py:52-185);
* RMSNorm computed in fp32, with the residual add fused as in
  nanovllm/layers/layernorm.py:17-44 (the bf16 sum becomes the next
  residual);
* SiLU(gate) * up;
* an LM head tied to the embedding unless the config says otherwise.

Attention is ``nanokv_amd.attention.Attention``: the M12 runtime on this
library's kernels, routed by the per-step context.  On the GPU the
elementwise chains are this library's fused kernels (nkv_rmsnorm,
nkv_qk_norm_rope, nkv_silu_mul: one launch each, same rounding points) and
the decode-step projections its HBM-bound GEMV (nkv_gemv); the tensor-op
formulas below are the CPU path of the same modules.

Weights come from a local checkpoint directory (config.json + *.safetensors
with the Hugging Face Qwen3 parameter names, packed into the fused
projections as nanovllm/utils/loader.py:12-28 does) or are random-initialised
for measurement (``init_random_``).  ``prefill`` / ``decode`` drive the model
the way the reference's ModelRunner does for one sequence: prefill in chunks
(the first chunk dense within itself, later chunks sparse), then one token
per decode step.
"""

from __future__ import annotations

import glob
import json
import math
import os
from dataclasses import dataclass, fields

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from .attention import Attention, attach_m12_runtimes, set_context
from .sparse.m12_runtime import M12Config
from .store import _ptr, _stream


def _fused(t: torch.Tensor) -> bool:
    """GPU bf16 tensors take the fused kernels (the library must load)."""
    return t.is_cuda and t.dtype == torch.bfloat16


def rmsnorm_dev(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None):
    """nkv_rmsnorm over the last dim: y, or (y, bf16(x + residual)) with a residual."""
    x = x.contiguous()
    n = x.shape[-1]
    out = torch.empty_like(x)
    res_out = None
    if residual is not None:
        residual = residual.contiguous()
        res_out = torch.empty_like(x)
    _lib.check(_lib.load().nkv_rmsnorm(_ptr(x), _ptr(residual), _ptr(weight.contiguous()), _ptr(out), _ptr(res_out),
                                       x.numel() // n, n, float(eps), _stream()), "rmsnorm")
    return out if residual is None else (out, res_out)


def qk_norm_rope_dev(qkv: torch.Tensor, positions: torch.Tensor, hq: int, hkv: int, q_weight, k_weight,
                     eps: float, cos: torch.Tensor, sin: torch.Tensor):
    """nkv_qk_norm_rope: qkv [T, (Hq + 2 Hkv) * 128] -> q [T, Hq, 128], k, v [T, Hkv, 128]."""
    qkv = qkv.contiguous()
    T = qkv.shape[0]
    q = torch.empty(T, hq, 128, dtype=qkv.dtype, device=qkv.device)
    k = torch.empty(T, hkv, 128, dtype=qkv.dtype, device=qkv.device)
    v = torch.empty_like(k)
    pos = positions.to(torch.int64).contiguous()
    _lib.check(_lib.load().nkv_qk_norm_rope(_ptr(qkv), T, hq, hkv, _ptr(q_weight.contiguous()),
                                            _ptr(k_weight.contiguous()), _ptr(cos), _ptr(sin), cos.shape[0],
                                            _ptr(pos), float(eps), _ptr(q), _ptr(k), _ptr(v), _stream()),
               "qk_norm_rope")
    return q, k, v


def _check_gemv_operands(x: torch.Tensor, weight: torch.Tensor, who: str) -> None:
    """The GEMV kernels read weight as a dense [n, k] bf16 matrix on x's device."""
    if x.dim() != 2 or not 1 <= x.shape[0] <= 4 or x.shape[1] % 8:
        raise ValueError(f"{who}: x must be [m, k] with 1 <= m <= 4 and k a multiple of 8 (got {tuple(x.shape)})")
    if weight.dim() != 2 or weight.shape[1] != x.shape[1]:
        raise ValueError(f"{who}: weight must be [n, {x.shape[1]}] (got {tuple(weight.shape)})")
    if weight.device != x.device or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError(f"{who}: x and weight must be bfloat16 tensors on one device")
    if not weight.is_contiguous():
        raise ValueError(f"{who}: weight must be contiguous")


def gemv_dev(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """nkv_gemv: x [m, k] (1 <= m <= 4) . weight [n, k]^T -> [m, n]."""
    x = x.contiguous()
    _check_gemv_operands(x, weight, "gemv")
    m, k = x.shape
    n = weight.shape[0]
    y = torch.empty(m, n, dtype=x.dtype, device=x.device)
    _lib.check(_lib.load().nkv_gemv(_ptr(weight), _ptr(x), _ptr(y), m, n, k, _stream()), "gemv")
    return y


def gemv_silu_mul_dev(x: torch.Tensor, gate_up_weight: torch.Tensor) -> torch.Tensor:
    """nkv_gemv_silu_mul: x [m, k] (1 <= m <= 4), gate|up weight [2 I, k] -> SiLU(gate) * up [m, I]."""
    x = x.contiguous()
    _check_gemv_operands(x, gate_up_weight, "gemv_silu_mul")
    if gate_up_weight.shape[0] % 2:
        raise ValueError("gemv_silu_mul: the gate|up weight needs an even number of rows")
    m, k = x.shape
    inter = gate_up_weight.shape[0] // 2
    y = torch.empty(m, inter, dtype=x.dtype, device=x.device)
    _lib.check(_lib.load().nkv_gemv_silu_mul(_ptr(gate_up_weight), _ptr(x), _ptr(y), m, inter, k, _stream()),
               "gemv_silu_mul")
    return y


def _gemv_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    return (_fused(x) and x.dim() == 2 and 1 <= x.shape[0] <= 4 and x.shape[1] % 8 == 0
            and weight.dim() == 2 and weight.shape[1] == x.shape[1] and weight.device == x.device
            and weight.dtype == torch.bfloat16 and weight.is_contiguous())


def prefill_chunk_bounds(n: int, chunk: int) -> list:
    """[(start, end)] of the prefill chunks of an n-token prompt, none shorter
    than 2 tokens (the store appends chunks of at least two tokens,
    m12_runtime.py:420-431): a 1-token tail takes one token from the chunk
    before it (chunks of 2 merge into one of 3).  Raises ValueError for
    prompts of fewer than 2 tokens, before anything runs."""
    if chunk < 2:
        raise ValueError(f"the prefill chunk must be at least 2 tokens (got {chunk})")
    if n < 2:
        raise ValueError(f"a prompt needs at least 2 tokens (got {n})")
    ends = list(range(chunk, n, chunk)) + [n]
    if len(ends) > 1 and ends[-1] - ends[-2] == 1:
        if chunk > 2:
            ends[-2] -= 1
        else:
            del ends[-2]
    starts = [0] + ends[:-1]
    return list(zip(starts, ends))


class Linear(nn.Linear):
    """nn.Linear whose products of 1-4 rows on the GPU (decode steps) run on
    nkv_gemv; longer inputs (prefill) stay on the library GEMM."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.bias is None and _gemv_ok(x, self.weight):
            return gemv_dev(x, self.weight)
        return F.linear(x, self.weight, self.bias)


def silu_mul_dev(gate_up: torch.Tensor) -> torch.Tensor:
    """nkv_silu_mul: [T, 2 I] (gate | up) -> [T, I]."""
    gate_up = gate_up.contiguous()
    inter = gate_up.shape[-1] // 2
    out = torch.empty(*gate_up.shape[:-1], inter, dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(_lib.load().nkv_silu_mul(_ptr(gate_up), _ptr(out), gate_up.numel() // (2 * inter), inter, _stream()),
               "silu_mul")
    return out


@dataclass
class Qwen3Config:
    """The fields of a Hugging Face Qwen3 config.json the decoder reads
    (defaults: Qwen3-4B)."""
    vocab_size: int = 151936
    hidden_size: int = 2560
    intermediate_size: int = 9728
    num_hidden_layers: int = 36
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    attention_bias: bool = False
    hidden_act: str = "silu"
    rope_scaling: dict | None = None

    def __post_init__(self):
        if self.hidden_act != "silu":
            raise ValueError(f"hidden_act {self.hidden_act!r} is not supported (silu only)")
        if isinstance(self.rope_scaling, dict):
            kind = self.rope_scaling.get("rope_type", self.rope_scaling.get("type"))
            if kind not in (None, "default", "yarn"):
                raise ValueError(f"rope_scaling type {kind!r} is not supported (plain RoPE or yarn)")
            self.rope_theta = float(self.rope_scaling.get("rope_theta", self.rope_theta))
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")

    @property
    def yarn(self) -> tuple | None:
        """(factor, original max positions, beta_fast, beta_slow, attention factor, truncate)
        for a YaRN config, else None."""
        r = self.rope_scaling
        if not isinstance(r, dict) or r.get("rope_type", r.get("type")) != "yarn":
            return None
        factor = float(r.get("factor", 1.0))
        att = r.get("attention_factor")
        return (factor, int(r.get("original_max_position_embeddings", self.max_position_embeddings)),
                float(r.get("beta_fast", 32.0)), float(r.get("beta_slow", 1.0)),
                yarn_attention_factor(factor) if att is None else float(att), bool(r.get("truncate", True)))

    @classmethod
    def from_dir(cls, path: str) -> "Qwen3Config":
        with open(os.path.join(path, "config.json")) as f:
            raw = json.load(f)
        names = {fd.name for fd in fields(cls)}
        return cls(**{k: v for k, v in raw.items() if k in names})


class RMSNorm(nn.Module):
    """y = bf16(x * rsqrt(mean(x^2) + eps)) * w with the statistics in fp32.

    With a residual, x is first replaced by the fp32 sum x + residual, whose
    bf16 rounding is returned as the new residual
    (nanovllm/layers/layernorm.py:17-44)."""

    def __init__(self, n: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(n))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if _fused(x) and self.weight.dtype == torch.bfloat16 and x.shape[-1] % 8 == 0:
            return rmsnorm_dev(x, self.weight, self.eps, residual)
        xf = x.float()
        if residual is not None:
            xf = xf + residual.float()
            residual = xf.to(x.dtype)
        y = (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight
        return y if residual is None else (y, residual)


_ROPE_TABLES: dict = {}


def yarn_attention_factor(factor: float) -> float:
    """YaRN's cos/sin scale: 0.1 ln(s) + 1 for s > 1 (Peng et al., 2023)."""
    return 1.0 if factor <= 1.0 else 0.1 * math.log(factor) + 1.0


def yarn_inv_freq(head_dim: int, base: float, factor: float, original_max: int, beta_fast: float = 32.0,
                  beta_slow: float = 1.0, truncate: bool = True) -> torch.Tensor:
    """YaRN inverse frequencies (Peng et al., 2023, "YaRN: Efficient Context
    Window Extension of Large Language Models"): dimension pair i rotates at
    base^(-2i/D) (extrapolation) for the fast pairs, at that over `factor`
    (interpolation) for the slow ones, and a linear ramp in between.  The
    ramp runs over the pairs whose wavelength at `original_max` positions
    makes between beta_fast and beta_slow turns: the pair index that turns
    `rot` times is D ln(original_max / (2 pi rot)) / (2 ln base)."""
    pos_freq = base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    extrap = 1.0 / pos_freq
    interp = 1.0 / (factor * pos_freq)

    def pair_for(rot: float) -> float:
        return head_dim * math.log(original_max / (2.0 * math.pi * rot)) / (2.0 * math.log(base))

    lo, hi = pair_for(beta_fast), pair_for(beta_slow)
    if truncate:
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0), min(hi, head_dim - 1)
    if lo == hi:
        hi += 0.001
    ramp = ((torch.arange(head_dim // 2, dtype=torch.float32) - lo) / (hi - lo)).clamp(0.0, 1.0)
    return interp * ramp + extrap * (1.0 - ramp)


def _rope_table(head_dim: int, base: float, max_position: int, device, yarn: tuple | None = None) -> tuple:
    """cos / sin [max_position, head_dim / 2] fp32 on `device` (times YaRN's
    attention factor with `yarn`), shared by every layer (built once per shape,
    scaling and device)."""
    key = (head_dim, float(base), max_position, yarn, str(torch.device(device)))
    t = _ROPE_TABLES.get(key)
    if t is None:
        if yarn is None:
            inv_freq, att = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)), 1.0
        else:
            factor, orig, bf, bs, att, trunc = yarn
            inv_freq = yarn_inv_freq(head_dim, base, factor, orig, bf, bs, trunc)
        ang = torch.arange(max_position, dtype=torch.float32)[:, None] * inv_freq[None, :]
        cos, sin = ang.cos(), ang.sin()
        if att != 1.0:
            cos, sin = cos * att, sin * att
        t = _ROPE_TABLES[key] = (cos.to(device), sin.to(device))
    return t


class RotaryEmbedding(nn.Module):
    """Rotate-half RoPE over the whole head: dims i and i + D/2 form a pair
    rotated by the angle pos * base^(-2i/D), in fp32
    (nanovllm/layers/rotary_embedding.py:6-50).  The tables are not module
    state, so casting the model to bf16 leaves them fp32."""

    def __init__(self, head_dim: int, base: float, max_position: int, yarn: tuple | None = None):
        super().__init__()
        self.head_dim, self.base, self.max_position, self.yarn = head_dim, base, max_position, yarn

    def table(self, device) -> tuple:
        return _rope_table(self.head_dim, self.base, self.max_position, device, self.yarn)

    def forward(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor):
        cos, sin = self.table(positions.device)
        cos = cos[positions].unsqueeze(1)   # [T, 1, D/2]
        sin = sin[positions].unsqueeze(1)
        return _rotate(q, cos, sin), _rotate(k, cos, sin)


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    a, b = x.float().chunk(2, dim=-1)
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1).to(x.dtype)


class Qwen3Attention(nn.Module):
    def __init__(self, cfg: Qwen3Config, max_position: int):
        super().__init__()
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = cfg.head_dim
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = Linear(cfg.hidden_size, self.q_size + 2 * self.kv_size, bias=cfg.attention_bias)
        self.o_proj = Linear(self.q_size, cfg.hidden_size, bias=False)
        self.qk_norm = not cfg.attention_bias
        if self.qk_norm:
            self.q_norm = RMSNorm(self.head_dim, cfg.rms_norm_eps)
            self.k_norm = RMSNorm(self.head_dim, cfg.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(self.head_dim, cfg.rope_theta, max_position, cfg.yarn)
        self.attn = Attention(self.num_heads, self.head_dim, self.head_dim ** -0.5, self.num_kv_heads)

    def forward(self, positions: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
        qkv = self.qkv_proj(h)
        if self.qk_norm and self.head_dim == 128 and _fused(qkv):
            cos, sin = self.rotary_emb.table(qkv.device)
            q, k, v = qk_norm_rope_dev(qkv, positions, self.num_heads, self.num_kv_heads, self.q_norm.weight,
                                       self.k_norm.weight, self.q_norm.eps, cos, sin)
            return self.o_proj(self.attn(q, k, v).flatten(1))
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = q.reshape(-1, self.num_heads, self.head_dim)
        k = k.reshape(-1, self.num_kv_heads, self.head_dim)
        v = v.reshape(-1, self.num_kv_heads, self.head_dim)
        if self.qk_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)
        q, k = self.rotary_emb(positions, q, k)
        o = self.attn(q, k, v.contiguous())
        return self.o_proj(o.flatten(1))


class Qwen3MLP(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.intermediate_size = cfg.intermediate_size
        self.gate_up_proj = Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if (self.gate_up_proj.bias is None and _gemv_ok(x, self.gate_up_proj.weight)
                and self.gate_up_proj.weight.shape[0] % 2 == 0):
            return self.down_proj(gemv_silu_mul_dev(x, self.gate_up_proj.weight))   # one launch for both
        gu = self.gate_up_proj(x)
        if _fused(gu) and self.intermediate_size % 8 == 0:
            return self.down_proj(silu_mul_dev(gu))
        gate, up = gu.split(self.intermediate_size, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen3Config, max_position: int):
        super().__init__()
        self.self_attn = Qwen3Attention(cfg, max_position)
        self.mlp = Qwen3MLP(cfg)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, positions, h, residual):
        if residual is None:
            h, residual = self.input_layernorm(h), h
        else:
            h, residual = self.input_layernorm(h, residual)
        h = self.self_attn(positions, h)
        h, residual = self.post_attention_layernorm(h, residual)
        return self.mlp(h), residual


class Qwen3Model(nn.Module):
    def __init__(self, cfg: Qwen3Config, max_position: int):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Qwen3DecoderLayer(cfg, max_position) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        h = self.embed_tokens(input_ids)
        residual = None
        for layer in self.layers:
            h, residual = layer(positions, h, residual)
        h, _ = self.norm(h, residual)
        return h


class Qwen3ForCausalLM(nn.Module):
    """Qwen3 causal LM (nanovllm/models/qwen3.py:186-220) with sparse attention.

    ``max_position`` sizes the RoPE tables (at least the longest sequence the
    model will see)."""

    def __init__(self, cfg: Qwen3Config, max_position: int | None = None):
        super().__init__()
        self.config = cfg
        self.max_position = max(max_position or 0, cfg.max_position_embeddings)
        if cfg.yarn is not None:   # the extended context YaRN is configured for
            self.max_position = max(self.max_position, int(cfg.yarn[1] * cfg.yarn[0]))
        self.model = Qwen3Model(cfg, self.max_position)
        if cfg.tie_word_embeddings:
            self.lm_head_weight = self.model.embed_tokens.weight
        else:
            self.lm_head_weight = nn.Parameter(torch.empty(cfg.vocab_size, cfg.hidden_size))
        self.requires_grad_(False)   # inference only
        self.runtimes = []
        self._graph = None       # captured decode step (decode_graph)
        self._graph_io = None    # its (token, position, logits) buffers
        self._graph_warm = False

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        return self.model(input_ids, positions)

    def compute_logits(self, h: torch.Tensor) -> torch.Tensor:
        if _gemv_ok(h, self.lm_head_weight):
            return gemv_dev(h, self.lm_head_weight)
        return F.linear(h, self.lm_head_weight)

    # -- sparse runtime wiring and one-sequence driving -------------------------
    def attach(self, m12: M12Config, device=None) -> list:
        """One M12 runtime per layer over one shared HBM store (model_runner.py:125-183)."""
        c = self.config
        if (m12.num_heads, m12.num_kv_heads, m12.head_dim) != (c.num_attention_heads, c.num_key_value_heads,
                                                               c.head_dim):
            raise ValueError("M12Config head shape differs from the model's")
        if m12.max_model_len > self.max_position:
            raise ValueError(f"max_model_len {m12.max_model_len} exceeds the RoPE table ({self.max_position})")
        self.runtimes = attach_m12_runtimes(self, m12, device)
        return self.runtimes

    def reset(self) -> None:
        self.release_graph()
        for rt in self.runtimes:
            rt.reset()

    def release_graph(self) -> None:
        """Drop the captured decode step (it holds this sequence's sizes and buffers)."""
        self._graph = self._graph_io = None
        self._graph_warm = False
        for rt in self.runtimes:
            rt.device_ring = False

    @torch.inference_mode()
    def prefill(self, input_ids: torch.Tensor, chunk: int = 4096) -> torch.Tensor:
        """Prefill a new sequence in chunks of `chunk` tokens; returns the
        logits of its last token ([vocab] fp32)."""
        if not self.runtimes:
            raise RuntimeError("attach() the sparse runtimes first")
        if self.runtimes[0].valid_len:
            raise RuntimeError("prefill starts a new sequence: reset() first")
        self.release_graph()
        n = input_ids.numel()
        if n > self.max_position:
            raise ValueError(f"prompt of {n} tokens exceeds the RoPE table ({self.max_position})")
        bounds = prefill_chunk_bounds(n, chunk)
        h = None
        for s, e in bounds:
            ids = input_ids[s:e]
            pos = torch.arange(s, e, device=ids.device)
            set_context(True, max_seqlen_q=ids.numel(), max_seqlen_k=s + ids.numel())
            h = self(ids, pos)
        return self.compute_logits(h[-1:]).float()[0]

    @torch.inference_mode()
    def decode(self, token: torch.Tensor, position: int) -> torch.Tensor:
        """One decode step for token ([1] int64) at `position`; returns its logits."""
        if not 0 <= position < self.max_position:
            raise ValueError(f"position {position} outside the RoPE table ({self.max_position})")
        set_context(False, max_seqlen_q=1)
        pos = torch.full((1,), position, dtype=torch.long, device=token.device)
        return self.compute_logits(self(token, pos)).float()[0]

    @torch.inference_mode()
    def decode_graph(self, token: torch.Tensor, position: int) -> torch.Tensor:
        """decode() with the whole token step captured in a HIP graph.

        For steady decode (every layer's sink and recent window full and the
        default decode selection): the first call runs eagerly through the
        device-ring entry (which also allocates every workspace), the second
        captures the step (embedding, every layer's dense ops and sparse
        layer-step, final norm, LM head) and replays it, and later calls only
        replay.  The selection sizes of this sequence are part of the graph,
        so reset() / prefill() drop it.  The returned logits are the graph's
        output buffer: the next call overwrites them."""
        if not self.runtimes:
            raise RuntimeError("attach() the sparse runtimes first")
        if not 0 <= position < self.max_position:
            raise ValueError(f"position {position} outside the RoPE table ({self.max_position})")
        if not all(rt.device_ring_ready() for rt in self.runtimes):
            raise RuntimeError("decode_graph needs a full sink and recent window and the default decode "
                               "selection (use decode() until then)")
        for rt in self.runtimes:
            rt.device_ring = True
        if self._graph is None:
            if not self._graph_warm:
                self._graph_warm = True
                return self.decode(token, position)
            self._capture(token.device)
        tok, pos, logits = self._graph_io
        tok.copy_(token.view(1))
        pos.fill_(position)
        self._graph.replay()
        for rt in self.runtimes:
            rt.ring_replayed()
        return logits

    def _capture(self, device) -> None:
        tok = torch.zeros(1, dtype=torch.long, device=device)
        pos = torch.zeros(1, dtype=torch.long, device=device)
        states = [rt.decode_state() for rt in self.runtimes]
        set_context(False, max_seqlen_q=1)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            logits = self.compute_logits(self(tok, pos)).float()[0]
        for rt, st in zip(self.runtimes, states):   # capturing ran no step
            rt.restore_decode_state(st)
        self._graph, self._graph_io = g, (tok, pos, logits)

    @torch.inference_mode()
    def generate_greedy(self, prompt: torch.Tensor, max_new_tokens: int, chunk: int = 4096) -> list:
        logits = self.prefill(prompt, chunk)
        out = []
        pos = prompt.numel()
        for _ in range(max_new_tokens):
            tok = logits.argmax().view(1)
            out.append(int(tok))
            logits = self.decode(tok, pos)
            pos += 1
        return out


# -- weights -------------------------------------------------------------------
def _packed_target(model: Qwen3ForCausalLM, name: str):
    """(parameter, row offset) for a Hugging Face name that lands in a fused
    projection (q/k/v -> qkv_proj, gate/up -> gate_up_proj), else None."""
    c = model.config
    q, kv = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
    offs = {"q_proj": ("qkv_proj", 0), "k_proj": ("qkv_proj", q), "v_proj": ("qkv_proj", q + kv),
            "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", c.intermediate_size)}
    for part, (fused, off) in offs.items():
        if f".{part}." in name:
            return model.get_parameter(name.replace(f".{part}.", f".{fused}.")), off
    return None


@torch.no_grad()
def load_checkpoint(model: Qwen3ForCausalLM, path: str) -> int:
    """Copy every tensor of the *.safetensors files under `path` into `model`
    (Hugging Face Qwen3 names); returns the number of tensors loaded.  Unknown
    names and shape mismatches raise."""
    from safetensors import safe_open

    files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors under {path}")
    n = 0
    for fn in files:
        with safe_open(fn, framework="pt", device="cpu") as f:
            for name in f.keys():
                t = f.get_tensor(name)
                if name == "lm_head.weight":
                    model.lm_head_weight.copy_(t)
                else:
                    tgt = _packed_target(model, name)
                    if tgt is not None:
                        p, off = tgt
                        p[off:off + t.shape[0]].copy_(t)
                    else:
                        p = model.get_parameter(name)
                        if p.shape != t.shape:
                            raise ValueError(f"{name}: checkpoint shape {tuple(t.shape)} != {tuple(p.shape)}")
                        p.copy_(t)
                n += 1
    return n


@torch.no_grad()
def init_random_(model: Qwen3ForCausalLM, seed: int = 0, std: float = 0.02) -> None:
    """N(0, std) matrices and embeddings, unit norms, zero biases (for
    measurement without a checkpoint)."""
    g = None
    for name, p in model.named_parameters():
        if g is None or g.device != p.device:
            g = torch.Generator(device=p.device).manual_seed(seed)
        if name.endswith("norm.weight"):
            p.fill_(1.0)
        elif name.endswith(".bias"):
            p.zero_()
        else:
            p.copy_(torch.randn(p.shape, generator=g, device=p.device, dtype=torch.float32) * std)


def from_pretrained(path: str, m12: M12Config | None = None, device="cuda",
                    dtype=torch.bfloat16) -> Qwen3ForCausalLM:
    """Build from a local checkpoint directory and attach the sparse runtimes."""
    cfg = Qwen3Config.from_dir(path)
    m12 = m12 or M12Config(num_heads=cfg.num_attention_heads, num_kv_heads=cfg.num_key_value_heads,
                           head_dim=cfg.head_dim)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)      # built in the target dtype: half the host memory of fp32
    try:
        model = Qwen3ForCausalLM(cfg, m12.max_model_len)
    finally:
        torch.set_default_dtype(prev)
    load_checkpoint(model, path)
    model.to(device=device, dtype=dtype)
    model.attach(m12, device)
    return model


__all__ = ["Qwen3Config", "Qwen3ForCausalLM", "RMSNorm", "RotaryEmbedding", "from_pretrained",
           "init_random_", "load_checkpoint"]
