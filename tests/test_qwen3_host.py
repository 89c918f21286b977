"""Host-side pieces of the Qwen3 decoder (no GPU): checkpoint packing, RoPE
and RMSNorm against their definitions, config handling."""

import json
import math

import pytest
import torch

from nanokv_amd.qwen3 import (Qwen3Config, Qwen3ForCausalLM, RMSNorm, RotaryEmbedding, init_random_,
                              load_checkpoint)
from nanokv_amd.sparse import M12Config

TINY = dict(vocab_size=64, hidden_size=256, intermediate_size=384, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)


def _hf_checkpoint(cfg, seed=0):
    """Tensors under the Hugging Face Qwen3 names (separate q/k/v, gate/up)."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    H, D, hq, hkv, I = cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads, \
        cfg.intermediate_size
    t = {"model.embed_tokens.weight": r(cfg.vocab_size, H), "model.norm.weight": r(H)}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        t.update({p + "self_attn.q_proj.weight": r(hq * D, H), p + "self_attn.k_proj.weight": r(hkv * D, H),
                  p + "self_attn.v_proj.weight": r(hkv * D, H), p + "self_attn.o_proj.weight": r(H, hq * D),
                  p + "self_attn.q_norm.weight": r(D), p + "self_attn.k_norm.weight": r(D),
                  p + "mlp.gate_proj.weight": r(I, H), p + "mlp.up_proj.weight": r(I, H),
                  p + "mlp.down_proj.weight": r(H, I), p + "input_layernorm.weight": r(H),
                  p + "post_attention_layernorm.weight": r(H)})
    return t


def test_checkpoint_packs_fused_projections(tmp_path):
    from safetensors.torch import save_file

    cfg = Qwen3Config(**TINY)
    t = _hf_checkpoint(cfg)
    names = sorted(t)
    save_file({k: t[k] for k in names[: len(names) // 2]}, str(tmp_path / "a.safetensors"))
    save_file({k: t[k] for k in names[len(names) // 2:]}, str(tmp_path / "b.safetensors"))
    model = Qwen3ForCausalLM(cfg)
    assert load_checkpoint(model, str(tmp_path)) == len(t)
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        qkv = model.get_parameter(p + "self_attn.qkv_proj.weight")
        assert torch.equal(qkv, torch.cat([t[p + f"self_attn.{x}_proj.weight"] for x in "qkv"]))
        gu = model.get_parameter(p + "mlp.gate_up_proj.weight")
        assert torch.equal(gu, torch.cat([t[p + "mlp.gate_proj.weight"], t[p + "mlp.up_proj.weight"]]))
        for name in ("self_attn.o_proj.weight", "self_attn.q_norm.weight", "mlp.down_proj.weight",
                     "post_attention_layernorm.weight"):
            assert torch.equal(model.get_parameter(p + name), t[p + name])
    # tied head: the embedding is the LM head
    assert torch.equal(model.lm_head_weight, t["model.embed_tokens.weight"])


def test_checkpoint_rejects_unknown_names_and_shapes(tmp_path):
    from safetensors.torch import save_file

    cfg = Qwen3Config(**TINY)
    save_file({"model.layers.0.self_attn.o_proj.weight": torch.zeros(3, 3)}, str(tmp_path / "x.safetensors"))
    with pytest.raises(ValueError, match="o_proj"):
        load_checkpoint(Qwen3ForCausalLM(cfg), str(tmp_path))
    save_file({"model.nonexistent.weight": torch.zeros(3)}, str(tmp_path / "x.safetensors"))
    with pytest.raises(AttributeError):
        load_checkpoint(Qwen3ForCausalLM(cfg), str(tmp_path))
    with pytest.raises(FileNotFoundError):
        load_checkpoint(Qwen3ForCausalLM(cfg), str(tmp_path / "empty"))


def test_rope_known_answer_identity_and_relative_position():
    # D = 4, base 100: pairs (0, 2) at angle p * 1, (1, 3) at angle p * 0.1
    rope = RotaryEmbedding(4, 100.0, 64)
    x = torch.tensor([[[1.0, 2.0, 3.0, 4.0]]])
    q1, _ = rope(torch.tensor([1]), x, x)
    c1, s1, c2, s2 = math.cos(1), math.sin(1), math.cos(0.1), math.sin(0.1)
    want = [1 * c1 - 3 * s1, 2 * c2 - 4 * s2, 3 * c1 + 1 * s1, 4 * c2 + 2 * s2]
    assert torch.allclose(q1[0, 0].double(), torch.tensor(want, dtype=torch.float64), atol=1e-6)
    q0, _ = rope(torch.tensor([0]), x, x)
    assert torch.equal(q0, x)                                 # position 0 rotates nothing
    # scores depend on the position difference only; each pair keeps its norm
    rope = RotaryEmbedding(128, 1e6, 4096)
    g = torch.Generator().manual_seed(0)
    q, k = torch.randn(1, 1, 128, generator=g), torch.randn(1, 1, 128, generator=g)
    dots = []
    for m, n in ((5, 2), (105, 102), (3000, 2997)):
        qm, _ = rope(torch.tensor([m]), q, q)
        _, kn = rope(torch.tensor([n]), k, k)
        dots.append(float((qm * kn).sum()))
        pair = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2  # noqa: E731
        assert torch.allclose(pair(qm), pair(q), rtol=1e-5, atol=1e-6)
    assert max(dots) - min(dots) <= 1e-3 * abs(dots[0]) + 1e-4


def test_rmsnorm_known_answer_and_residual():
    n = RMSNorm(2, eps=0.0)
    with torch.no_grad():
        n.weight.copy_(torch.tensor([1.0, 2.0]))
    x = torch.tensor([[3.0, 4.0]])
    y = n(x)
    s = math.sqrt(12.5)
    assert torch.allclose(y, torch.tensor([[3 / s, 8 / s]]))
    y2, res = n(torch.tensor([[1.0, 1.0]]), torch.tensor([[2.0, 3.0]]))
    assert torch.equal(res, torch.tensor([[3.0, 4.0]])) and torch.allclose(y2, y)
    xb = torch.tensor([[3.0, 4.0]], dtype=torch.bfloat16)
    assert n.to(torch.bfloat16)(xb).dtype == torch.bfloat16


def test_config_from_dir_and_unsupported_variants(tmp_path):
    raw = dict(TINY, architectures=["Qwen3ForCausalLM"], torch_dtype="bfloat16", rope_theta=5e5)
    (tmp_path / "config.json").write_text(json.dumps(raw))
    cfg = Qwen3Config.from_dir(str(tmp_path))
    assert cfg.hidden_size == 256 and cfg.rope_theta == 5e5 and cfg.tie_word_embeddings
    with pytest.raises(ValueError, match="rope_scaling"):
        Qwen3Config(rope_scaling={"rope_type": "longrope", "factor": 4.0})
    assert Qwen3Config(rope_scaling={"rope_type": "default", "rope_theta": 7.0}).rope_theta == 7.0
    with pytest.raises(ValueError, match="silu"):
        Qwen3Config(hidden_act="gelu")


def test_attach_checks_head_shape_and_rope_range():
    model = Qwen3ForCausalLM(Qwen3Config(**TINY))
    with pytest.raises(ValueError, match="head shape"):
        model.attach(M12Config(num_heads=32, num_kv_heads=8))
    with pytest.raises(ValueError, match="RoPE"):
        model.attach(M12Config(num_heads=4, num_kv_heads=2, max_model_len=1 << 20))
    with pytest.raises(RuntimeError, match="attach"):
        model.prefill(torch.zeros(4, dtype=torch.long))


def test_random_init_is_seeded():
    a, b = Qwen3ForCausalLM(Qwen3Config(**TINY)), Qwen3ForCausalLM(Qwen3Config(**TINY))
    init_random_(a, 3)
    init_random_(b, 3)
    assert all(torch.equal(x, y) for x, y in zip(a.parameters(), b.parameters()))
    assert torch.equal(a.model.norm.weight, torch.ones(256))
    assert 0.015 < float(a.model.layers[0].mlp.down_proj.weight.detach().std()) < 0.025
    assert not any(p.requires_grad for p in a.parameters())   # inference-only


def test_reference_model_detects_a_decode_position_off_by_one():
    """The float64 restatement the GPU end-to-end test compares against, with
    a mistake planted in it: decode RoPE at position + 1.  Its attention
    outputs and logits move by more than that test's tolerances (2%, 2.5%)."""
    from tests._qwen3_ref import RefQwen3

    class OffByOne(RefQwen3):
        def _rope(self, x, pos):
            return super()._rope(x, pos + (1 if pos.numel() == 1 else 0))

    cfg = Qwen3Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=4096)
    m12 = M12Config(max_model_len=2048, num_heads=8, num_kv_heads=2)
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, 7)
    state = model.to(torch.bfloat16).state_dict()
    prompt = torch.randint(0, cfg.vocab_size, (1024,), generator=torch.Generator().manual_seed(3))
    runs = []
    for cls in (RefQwen3, OffByOne):
        r = cls(state, cfg, m12)
        r.forward(prompt[:512], "first")
        r.forward(prompt[512:], "chunk")
        runs.append((r.forward(torch.tensor([127]), "decode")[-1], r.attn_out[-1]))
    rel = lambda a, b: float((a - b).norm() / b.norm())  # noqa: E731
    assert rel(runs[1][0], runs[0][0]) > 2 * 0.025
    for a, b in zip(runs[1][1], runs[0][1]):
        assert rel(torch.from_numpy(a), torch.from_numpy(b)) > 0.02


@pytest.mark.parametrize("factor,orig,theta,extra", [(4.0, 32768, 1e6, {}), (2.0, 4096, 1e4, {}),
                                                      (8.0, 8192, 5e5, {"beta_fast": 16, "beta_slow": 2}),
                                                      (4.0, 32768, 1e6, {"truncate": False})])
def test_yarn_matches_the_transformers_implementation(factor, orig, theta, extra):
    """YaRN inverse frequencies and attention factor against Hugging Face's
    own implementation (an independent restatement of the same paper)."""
    from transformers import Qwen3Config as HFQwen3Config
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    from nanokv_amd.qwen3 import yarn_attention_factor, yarn_inv_freq

    scaling = {"rope_type": "yarn", "factor": factor, "original_max_position_embeddings": orig, **extra}
    hf = HFQwen3Config(rope_scaling=dict(scaling, rope_theta=theta), rope_theta=theta, head_dim=128,
                       max_position_embeddings=int(orig * factor))
    inv_ref, att_ref = ROPE_INIT_FUNCTIONS["yarn"](hf, "cpu")
    inv = yarn_inv_freq(128, theta, factor, orig, float(extra.get("beta_fast", 32)),
                        float(extra.get("beta_slow", 1)), bool(extra.get("truncate", True)))
    assert torch.allclose(inv, inv_ref.float(), rtol=1e-6, atol=0)
    assert abs(yarn_attention_factor(factor) - att_ref) < 1e-12
    cfg = Qwen3Config(rope_theta=theta, rope_scaling=scaling, max_position_embeddings=orig)
    assert cfg.yarn[0] == factor and cfg.yarn[4] == pytest.approx(att_ref)
    assert Qwen3ForCausalLM(Qwen3Config(**dict(TINY, rope_scaling=scaling,
                                                max_position_embeddings=orig))).max_position >= orig * factor


def test_yarn_with_factor_one_is_plain_rope():
    from nanokv_amd.qwen3 import _rope_table

    plain = _rope_table(128, 1e6, 64, "cpu")
    yarn = _rope_table(128, 1e6, 64, "cpu", (1.0, 4096, 32.0, 1.0, 1.0, True))
    assert torch.allclose(plain[0], yarn[0], atol=1e-6) and torch.allclose(plain[1], yarn[1], atol=1e-6)


def test_prefill_chunk_plan_never_leaves_a_one_token_chunk():
    from nanokv_amd.qwen3 import prefill_chunk_bounds

    for n in range(2, 40):
        for chunk in range(2, 12):
            b = prefill_chunk_bounds(n, chunk)
            assert b[0][0] == 0 and b[-1][1] == n
            assert all(e0 == s1 for (_, e0), (s1, _) in zip(b, b[1:])), (n, chunk, b)
            assert all(e - s >= 2 for s, e in b), (n, chunk, b)
            assert all(e - s <= max(chunk, 3) for s, e in b), (n, chunk, b)
    assert prefill_chunk_bounds(4097, 4096) == [(0, 4095), (4095, 4097)]
    assert prefill_chunk_bounds(8192, 4096) == [(0, 4096), (4096, 8192)]
    with pytest.raises(ValueError):
        prefill_chunk_bounds(1, 4096)
    with pytest.raises(ValueError):
        prefill_chunk_bounds(100, 1)


def test_gemv_rejects_mismatched_weights_before_launching():
    from nanokv_amd.qwen3 import _gemv_ok, gemv_dev, gemv_silu_mul_dev

    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    for bad in (torch.zeros(16, 32, dtype=torch.bfloat16), torch.zeros(16, 64, dtype=torch.float32),
                torch.zeros(64, dtype=torch.bfloat16), torch.zeros(64, 16, dtype=torch.bfloat16).t()):
        assert not _gemv_ok(x, bad)
        with pytest.raises(ValueError):
            gemv_dev(x, bad)
    with pytest.raises(ValueError):
        gemv_silu_mul_dev(x, torch.zeros(15, 64, dtype=torch.bfloat16))
