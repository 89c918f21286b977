"""Float64 restatement of the Qwen3 decoder with the oracle's M12 attention.

Independent of nanokv_amd.qwen3: plain pre-norm residual stream,
RMSNorm / RoPE / SiLU written from their definitions in float64, and per
layer an oracle M12 layer (first chunk: dense causal attention within the
chunk, then store; later chunks: oracle prefill_chunk; decode: oracle decode).
Weights are read from a model's state_dict.
"""

import numpy as np
import torch

from oracle import nkv_oracle as O


class RefQwen3:
    def __init__(self, state: dict, cfg, m12):
        self.w = {k: v.detach().double().cpu() for k, v in state.items()}
        self.c = cfg
        self.layers = cfg.num_hidden_layers
        self.attn_out = []   # per call: [layer] -> o [T, Hq, D] float64
        oc = O.OracleConfig(block_size=m12.block_size, r=m12.r, recent_tokens=m12.recent_tokens,
                            sink_tokens=m12.sink_tokens, top_k_blocks=m12.top_k_blocks,
                            num_heads=cfg.num_attention_heads, num_kv_heads=cfg.num_key_value_heads,
                            head_dim=cfg.head_dim, scale=cfg.head_dim ** -0.5)
        self.oracles = [O.M12Oracle(oc) for _ in range(self.layers)]
        self.len = 0

    def _rms(self, x, w):
        return x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + self.c.rms_norm_eps) * w

    def _rope(self, x, pos):
        d = self.c.head_dim
        att = 1.0
        if self.c.yarn is None:
            inv = self.c.rope_theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
        else:   # Hugging Face's YaRN frequencies and attention factor
            from transformers import Qwen3Config as HFQwen3Config
            from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
            hf = HFQwen3Config(rope_scaling=dict(self.c.rope_scaling, rope_theta=self.c.rope_theta),
                               rope_theta=self.c.rope_theta, head_dim=d,
                               max_position_embeddings=self.c.max_position_embeddings)
            inv, att = ROPE_INIT_FUNCTIONS["yarn"](hf, "cpu")
            inv = inv.double()
        ang = pos.double()[:, None, None] * inv          # [T, 1, D/2]
        c, s = ang.cos() * att, ang.sin() * att
        a, b = x[..., : d // 2], x[..., d // 2:]
        return torch.cat((a * c - b * s, b * c + a * s), dim=-1)

    def forward(self, ids: torch.Tensor, phase: str) -> torch.Tensor:
        """ids [T]; phase 'first' | 'chunk' | 'decode'; returns logits [T, vocab] float64."""
        c, w = self.c, self.w
        T = ids.numel()
        pos = torch.arange(self.len, self.len + T)
        hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        r = w["model.embed_tokens.weight"][ids.cpu()]
        outs = []
        for i in range(self.layers):
            p = f"model.layers.{i}."
            x = self._rms(r, w[p + "input_layernorm.weight"])
            qkv = x @ w[p + "self_attn.qkv_proj.weight"].T
            q = qkv[:, : hq * d].reshape(T, hq, d)
            k = qkv[:, hq * d: (hq + hkv) * d].reshape(T, hkv, d)
            v = qkv[:, (hq + hkv) * d:].reshape(T, hkv, d)
            q = self._rms(q, w[p + "self_attn.q_norm.weight"])
            k = self._rms(k, w[p + "self_attn.k_norm.weight"])
            q, k = self._rope(q, pos), self._rope(k, pos)
            qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
            orc = self.oracles[i]
            if phase == "first":
                o = O.attention_fp64(qn, kn, vn, orc.cfg.scale, O.causal_mask(T, T, 0))
                orc.prefill_first(qn, kn, vn)
            elif phase == "chunk":
                _, o = orc.prefill_chunk(qn, kn, vn)
            else:
                _, _, o = orc.decode(qn, kn, vn)
            outs.append(np.asarray(o, np.float64))
            a = torch.from_numpy(np.asarray(o, np.float64)).reshape(T, hq * d) @ w[p + "self_attn.o_proj.weight"].T
            r = r + a
            x = self._rms(r, w[p + "post_attention_layernorm.weight"])
            gu = x @ w[p + "mlp.gate_up_proj.weight"].T
            g, u = gu[:, : c.intermediate_size], gu[:, c.intermediate_size:]
            r = r + (g * torch.sigmoid(g) * u) @ w[p + "mlp.down_proj.weight"].T
        self.attn_out.append(outs)
        self.len += T
        h = self._rms(r, w["model.norm.weight"])
        return h @ w["lm_head_weight"].T
