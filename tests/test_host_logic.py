"""Host-side logic of the runtime mirror (no GPU): config validation and the
reference's module-level helpers, with the reference tests' known answers."""

import pytest
import torch

from nanokv_amd.sparse import m12_runtime as rt
from oracle import nkv_oracle as O


@pytest.mark.parametrize("budget", [0, 33])
def test_prefill_budget_cannot_exceed_allocated_maximum(budget):
    # reference tests/test_m17_prefill_budget.py:9-12
    with pytest.raises(ValueError, match="prefill_top_k_blocks"):
        rt.M12Config(top_k_blocks=32, prefill_top_k_blocks=budget)


@pytest.mark.parametrize("budget", [0, 33])
def test_decode_budget_cannot_exceed_allocated_maximum(budget):
    # reference tests/test_m17_prefill_budget.py:66-69
    with pytest.raises(ValueError, match="decode_top_k_blocks"):
        rt.M12Config(top_k_blocks=32, decode_top_k_blocks=budget)


def test_pipeline_requires_direct_pinned_gather():
    # reference tests/test_m20_kv_pipeline.py:9-11
    with pytest.raises(ValueError, match="requires use_index_select"):
        rt.M12Config(use_index_select=False, decode_kv_pipeline=True)


@pytest.mark.parametrize("kw,msg", [
    ({"decode_relative_a": 1.5}, "decode_relative_a"),
    ({"decode_relative_a": 0.5, "decode_relative_max_blocks": 0}, "decode_relative_max_blocks"),
    ({"decode_query_window": 0}, "decode_query_window"),
    ({"fused_dequant": True}, "fused_dequant requires quant_history"),
    ({"quant_scale_layout": "row"}, "quant_scale_layout"),
    ({"attend_splits": 0}, "attend_splits"),
])
def test_config_validation_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        rt.M12Config(**kw)


def test_kv_format_mapping():
    assert rt.M12Config().kv_format == "bf16"
    assert rt.M12Config(quant_history=True).kv_format == "int8"
    assert rt.M12Config(quant_history=True, quant_scale_layout="token").kv_format == "int8_token"


def _split_choice(nseg, layers=36, kv_heads=8, nqg=1, rows=4, **cfg):
    from types import SimpleNamespace
    me = SimpleNamespace(cfg=rt.M12Config(**cfg), store=SimpleNamespace(num_kv_heads=kv_heads), nl=layers,
                         STREAM_MIN_SEGMENTS=rt._SparseCore.STREAM_MIN_SEGMENTS,
                         WIDE_PLAN_MIN_GROUPS=rt._SparseCore.WIDE_PLAN_MIN_GROUPS)
    return rt._SparseCore._splits(me, nseg, nqg, rows)


def test_decode_split_choice():
    # 36 layers x 8 KV heads, top-32 + sink + 8 recent pieces = 41 segments:
    # 11808 segments, the stream form (0) in every history format
    assert _split_choice(41) == 0
    assert _split_choice(41, quant_history=True) == 0
    assert _split_choice(41, quant_history=True, quant_scale_layout="token") == 0
    assert _split_choice(41, attend_splits=8) == 8             # explicit choice kept
    # below 4096 segments the split form: ~1440 workgroups (bf16), ~900 (int8),
    # at most one segment per wavefront (12 layers: 11 splits cap bf16's 15)
    assert _split_choice(41, layers=12) == 11
    assert _split_choice(41, layers=12, quant_history=True) == 9
    assert _split_choice(41, layers=13) == 0                   # 13 x 8 x 41 = 4264
    # verify: 6 draft tokens x 4 heads = 24 rows on the wide kernel, 16K history
    # (139 union blocks + sink + 8 recent pieces + the draft chunk = 149 segments)
    # 36 x 8 = 288 groups: the wide kernel's tiered plan (0); below 128
    # groups its ~900-workgroup split form
    assert _split_choice(149, rows=24) == 0
    assert _split_choice(149, rows=24, quant_history=True) == 0
    assert _split_choice(149, rows=24, layers=16) == 0          # 128 groups
    assert _split_choice(149, rows=24, layers=8) == 14          # 64 groups: ~900 workgroups
    assert _split_choice(149, rows=16) == 5                     # the 16-row kernel keeps ~1440
    for layers in range(1, 80):
        for nseg in (1, 5, 16, 41, 300):
            s = _split_choice(nseg, layers=layers)
            if layers * 8 * nseg >= 4096:
                assert s == 0                                    # the stream form
                continue
            assert 1 <= s <= max(1, min(-(-nseg // 4), 64))    # at most one segment per wavefront
            assert s == 1 or s % 4 != 0                          # never a multiple of 4
    assert _split_choice(16, layers=4) == 3                    # cap 4 is a multiple of 4: one less


@pytest.mark.parametrize("bad", [
    {"dtype": torch.float32}, {"head_dim": 64}, {"block_size": 32}, {"num_heads": 24}, {"r": 3},
])
def test_hip_runtime_rejects_shapes_the_kernels_do_not_cover(bad):
    with pytest.raises(ValueError):
        rt._check_hip_shapes(rt.M12Config(**bad))


def test_prefill_recent_slice_known_answers():
    # reference tests/test_m14_prefill_layout.py:34-44
    assert rt.prefill_recent_slice(4096, 64, 512) == (3584, 0, 512)
    assert rt.prefill_recent_slice(128, 64, 512) == (0, 64, 64)
    assert rt.prefill_recent_slice(64, 64, 512) == (0, 64, 0)
    for v in range(0, 1300, 37):
        assert rt.prefill_recent_slice(v, 64, 512) == O.prefill_recent_slice(v, 64, 512)


def test_dynamic_top_k_known_answers():
    # reference tests/test_m16_dynamic_topk.py:13-22
    f = rt.dynamic_top_k_from_scores
    assert f(torch.ones(32), 32, 0.90) == 32
    assert f(torch.arange(10, 0, -1).float(), 32, 0.90) == 10
    assert f(torch.tensor([float("inf")] + [0.0] * 31), 32, 0.90) == 32
    assert f(torch.tensor([10.0] + [0.0] * 31), 32, 0.90) == 16
    g = torch.Generator().manual_seed(3)
    for _ in range(50):
        s = torch.sort(torch.randn(32, generator=g) * 3, descending=True).values
        assert f(s, 32, 0.9) == O.dynamic_top_k_from_scores(s.numpy(), 32, 0.9)


class _FakeRuntime:
    """Records which runtime entry point Attention.forward calls."""

    def __init__(self, prefill_len=0):
        self.enabled = True
        self.verify_mode = False
        self.prefill_len = prefill_len
        self.calls = []

    def _rec(self, name, q):
        self.calls.append(name)
        return torch.full((q.shape[0], 1), float(len(self.calls)))

    def dense_prefill(self, q, k, v, scale=None):
        self.calls.append(("scale", scale))
        return self._rec("dense_prefill", q)

    def prefill_first(self, q, k, v):
        self.calls.append("prefill_first")
        self.prefill_len = q.shape[0]
        return {}

    def prefill_chunk(self, q, k, v, device=None):
        return self._rec("prefill_chunk", q)

    def decode(self, q, k, v, device=None):
        return self._rec("decode", q)

    def verify_tokens(self, q, k, v, device=None):
        return self._rec("verify_tokens", q)


def test_attention_routing_follows_the_reference_order():
    """nanovllm/layers/attention.py:64-99 sparse branch: verify, first chunk, later chunk, decode."""
    from nanokv_amd import attention as A

    layer = A.Attention(32, 128, 0.125, 8)
    fake = _FakeRuntime()
    layer.sparse_rt = fake
    q, k, v = torch.zeros(4, 32, 128), torch.zeros(4, 8, 128), torch.zeros(4, 8, 128)
    try:
        A.set_context(True, max_seqlen_q=4)
        layer(q, k, v)
        assert fake.calls == [("scale", 0.125), "dense_prefill", "prefill_first"]
        fake.calls.clear()
        layer(q, k, v)   # history exists now
        assert fake.calls == ["prefill_chunk"]
        fake.calls.clear()
        fake.verify_mode = True
        A.set_context(False)
        layer(q, k, v)   # verify ignores is_prefill and the token count
        assert fake.calls == ["verify_tokens"]
        fake.calls.clear()
        fake.verify_mode = False
        layer(q[:1], k[:1], v[:1])
        assert fake.calls == ["decode"]
        with pytest.raises(AssertionError, match="single query token"):
            layer(q, k, v)
        A.set_context(False, block_tables=torch.zeros(1, 1))
        with pytest.raises(AssertionError, match="block tables"):
            layer(q[:1], k[:1], v[:1])
        A.set_context(False)
        layer.k_cache = torch.zeros(3)
        with pytest.raises(AssertionError, match="zero paged blocks"):
            layer(q[:1], k[:1], v[:1])
    finally:
        A.reset_context()


def test_attention_without_runtime_raises():
    from nanokv_amd import attention as A

    layer = A.Attention(32, 128, 0.125, 8)
    with pytest.raises(NotImplementedError, match="sparse_rt"):
        layer(torch.zeros(1, 32, 128), torch.zeros(1, 8, 128), torch.zeros(1, 8, 128))
    fake = _FakeRuntime()
    fake.enabled = False
    layer.sparse_rt = fake
    with pytest.raises(NotImplementedError):
        layer(torch.zeros(1, 32, 128), torch.zeros(1, 8, 128), torch.zeros(1, 8, 128))


def test_context_mirrors_the_reference_fields():
    from nanokv_amd import attention as A

    assert list(A.Context.__dataclass_fields__) == [
        "is_prefill", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k",
        "slot_mapping", "context_lens", "block_tables"]
    A.set_context(True, None, None, 7)
    assert A.get_context().is_prefill and A.get_context().max_seqlen_q == 7
    A.reset_context()
    assert A.get_context() == A.Context()


def test_attach_requires_attention_modules():
    from nanokv_amd import attention as A

    with pytest.raises(ValueError, match="no attention modules"):
        A.attach_m12_runtimes(torch.nn.Linear(2, 2), rt.M12Config(max_model_len=1024))


@pytest.mark.parametrize("backend,msg", [
    ("flash", "expected explicit experimental backend"),       # segmented_prefill_adapter.py:60-61
    ("operator", "does not ship"),
])
def test_segmented_prefill_adapter_backend_errors(backend, msg):
    from nanokv_amd.sparse.segmented_prefill_adapter import SegmentedPrefillAdapter
    with pytest.raises(ValueError, match=msg):
        SegmentedPrefillAdapter(backend, 128 ** -0.5, (32, 8, 128, torch.bfloat16))
