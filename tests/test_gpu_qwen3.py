"""A whole Qwen3 decoder on the GPU with the sparse layer-step as its attention.

`nanokv_amd.qwen3.Qwen3ForCausalLM` (two layers, Hq=8, Hkv=2, D=128,
random weights) prefills 1024 tokens in two 512-token chunks (the first dense
within itself, the second through the sparse chunked prefill) and decodes
three tokens.  An independent float64 restatement (tests/_qwen3_ref.py:
RMSNorm, RoPE and SiLU from their definitions, the oracle's M12 attention per
layer) runs the same weights and tokens.

At 1024 tokens every selectable block is selected (16 blocks, 9 protected,
7 <= top-32), so the selections cannot differ between the bf16 and the
float64 paths and the comparison measures rounding only.

Tolerances: relative Frobenius error of every layer's attention output
<= 2% and of the logits <= 2.5%.  On the CPU the same bf16 module code with
the oracle's attention (outputs rounded to bf16) stays near 0.5% and 0.8%;
a decode RoPE position off by one moves the attention outputs by 4-13% and
the logits by 9%.
"""

import numpy as np
import pytest
import torch

from tests._qwen3_ref import RefQwen3
from tests._util import to_np

pytestmark = pytest.mark.gpu

ATTN_TOL, LOGIT_TOL = 0.02, 0.025


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("rope_scaling", [None, {"rope_type": "yarn", "factor": 8.0,
                                                  "original_max_position_embeddings": 256}])
def test_qwen3_prefill_and_decode_match_float64_reference(rope_scaling):
    """rope_scaling: plain RoPE, or YaRN with the 1027 positions of the test
    well past its original 256 (the reference restatement takes Hugging
    Face's YaRN frequencies)."""
    from nanokv_amd.qwen3 import Qwen3Config, Qwen3ForCausalLM, init_random_
    from nanokv_amd.sparse import M12Config

    cfg = Qwen3Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=256 if rope_scaling else 4096, rope_scaling=rope_scaling)
    m12 = M12Config(max_model_len=2048, num_heads=8, num_kv_heads=2)
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, 7)
    model = model.to(device="cuda", dtype=torch.bfloat16)
    ref = RefQwen3(model.state_dict(), cfg, m12)   # float64 copy of the bf16 weights
    rts = model.attach(m12)
    assert len(rts) == 2 and rts[0].store is rts[1].store

    caps = []
    for layer in model.model.layers:
        layer.self_attn.attn.register_forward_hook(lambda m, i, o: caps.append(to_np(o)))

    prompt = torch.randint(0, cfg.vocab_size, (1024,), generator=torch.Generator().manual_seed(3))
    print("prefill 2 x 512", flush=True)
    logits = model.prefill(prompt.cuda(), chunk=512)
    ref.forward(prompt[:512], "first")
    ref_logits = ref.forward(prompt[512:], "chunk")
    for i, o in enumerate(caps):
        e = _rel(o, ref.attn_out[i // 2][i % 2])
        print(f"prefill chunk {i // 2} layer {i % 2}: attention rel err {e:.4f}", flush=True)
        assert e <= ATTN_TOL
    e = _rel(to_np(logits), ref_logits[-1].numpy())
    print(f"prefill logits rel err {e:.4f}", flush=True)
    assert e <= LOGIT_TOL
    assert all(rt.prefill_len == 1024 and rt.nblocks_filled == 16 for rt in rts)

    pos = 1024
    for step in range(3):
        caps.clear()
        tok = logits.argmax().view(1)
        logits = model.decode(tok, pos)
        ref_logits = ref.forward(tok.cpu(), "decode")
        pos += 1
        for i, o in enumerate(caps):
            e = _rel(o, ref.attn_out[-1][i])
            assert e <= ATTN_TOL, f"decode {step} layer {i}: attention rel err {e:.4f}"
            assert sorted(rts[i].last_block_ids.tolist()) == sorted(ref.oracles[i].last_block_ids.tolist())
        e = _rel(to_np(logits), ref_logits[-1].numpy())
        print(f"decode {step}: logits rel err {e:.4f}", flush=True)
        assert e <= LOGIT_TOL
        assert all(rt.valid_len == 1024 + step + 1 for rt in rts)


def test_qwen3_decode_graph_replays_match_eager_decode():
    """decode_graph (one captured token step, replayed) against decode() of a
    twin model with the same weights and tokens: logits bit-identical on every
    step (the warm-up, the capturing step and 6 plain replays), with eager
    work and a synchronisation between replays."""
    from nanokv_amd.qwen3 import Qwen3Config, Qwen3ForCausalLM, init_random_
    from nanokv_amd.sparse import M12Config

    cfg = Qwen3Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=4096)
    m12 = M12Config(max_model_len=2048, num_heads=8, num_kv_heads=2)
    models = []
    for _ in range(2):
        m = Qwen3ForCausalLM(cfg)
        init_random_(m, 11)
        m = m.to(device="cuda", dtype=torch.bfloat16)
        m.attach(m12)
        models.append(m)
    eager, graphed = models
    prompt = torch.randint(0, cfg.vocab_size, (1024,), generator=torch.Generator().manual_seed(4)).cuda()
    la = eager.prefill(prompt, chunk=512)
    lb = graphed.prefill(prompt, chunk=512)
    assert torch.equal(la, lb)
    pos = 1024
    for step in range(8):
        tok = la.argmax().view(1)
        lb = graphed.decode_graph(tok, pos).clone()
        la = eager.decode(tok, pos)
        torch.cuda.synchronize()
        diff = float((la - lb).abs().max())
        print(f"step {step}: graph {'replay' if graphed._graph is not None else 'eager'}, max |diff| {diff:.3e}",
              flush=True)
        assert torch.equal(la, lb), f"step {step}: max |diff| {diff:.3e}"
        pos += 1
    assert [rt.valid_len for rt in graphed.runtimes] == [rt.valid_len for rt in eager.runtimes] == [1032] * 2
    graphed.reset()
    assert graphed._graph is None and not graphed.runtimes[0].device_ring


def test_from_pretrained_loads_a_local_checkpoint(tmp_path):
    """A checkpoint directory in the Hugging Face layout (config.json, two
    safetensors shards, separate q/k/v and gate/up tensors) through
    from_pretrained: prefill and decode logits equal those of the model built
    in memory from the same weights."""
    import json

    from safetensors.torch import save_file

    from nanokv_amd.qwen3 import Qwen3Config, Qwen3ForCausalLM, from_pretrained, init_random_
    from nanokv_amd.sparse import M12Config

    raw = dict(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
               num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
               tie_word_embeddings=True, architectures=["Qwen3ForCausalLM"], torch_dtype="bfloat16")
    (tmp_path / "config.json").write_text(json.dumps(raw))
    cfg = Qwen3Config.from_dir(str(tmp_path))
    ref = Qwen3ForCausalLM(cfg)
    init_random_(ref, 21)
    ref = ref.to(torch.bfloat16)
    q, kv, inter = 8 * 128, 2 * 128, 1024
    tensors = {"model.embed_tokens.weight": ref.model.embed_tokens.weight, "model.norm.weight": ref.model.norm.weight}
    for i, layer in enumerate(ref.model.layers):
        p = f"model.layers.{i}."
        qkv = layer.self_attn.qkv_proj.weight
        gu = layer.mlp.gate_up_proj.weight
        tensors.update({p + "self_attn.q_proj.weight": qkv[:q], p + "self_attn.k_proj.weight": qkv[q:q + kv],
                        p + "self_attn.v_proj.weight": qkv[q + kv:], p + "mlp.gate_proj.weight": gu[:inter],
                        p + "mlp.up_proj.weight": gu[inter:],
                        p + "self_attn.o_proj.weight": layer.self_attn.o_proj.weight,
                        p + "self_attn.q_norm.weight": layer.self_attn.q_norm.weight,
                        p + "self_attn.k_norm.weight": layer.self_attn.k_norm.weight,
                        p + "mlp.down_proj.weight": layer.mlp.down_proj.weight,
                        p + "input_layernorm.weight": layer.input_layernorm.weight,
                        p + "post_attention_layernorm.weight": layer.post_attention_layernorm.weight})
    names = sorted(tensors)
    for j, part in enumerate((names[: len(names) // 2], names[len(names) // 2:])):
        save_file({n: tensors[n].contiguous() for n in part}, str(tmp_path / f"model-{j}.safetensors"))

    m12 = M12Config(max_model_len=2048, num_heads=8, num_kv_heads=2)
    loaded = from_pretrained(str(tmp_path), m12)
    ref = ref.to("cuda")
    ref.attach(m12)
    prompt = torch.randint(0, 512, (700,), generator=torch.Generator().manual_seed(9)).cuda()
    la, lb = loaded.prefill(prompt, chunk=512), ref.prefill(prompt, chunk=512)
    assert torch.equal(la, lb)
    tok = la.argmax().view(1)
    assert torch.equal(loaded.decode(tok, 700), ref.decode(tok, 700))
