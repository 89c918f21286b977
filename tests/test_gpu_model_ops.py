"""The decoder's fused elementwise kernels against the tensor-op formulas
they replace (nanovllm/layers/layernorm.py:17-44,
nanovllm/layers/rotary_embedding.py:6-50, nanovllm/models/qwen3.py:99-110,
nanovllm/layers/activation.py:6-11), computed with torch on the same GPU.

Copies and sums that do not depend on a reduction order (v, the residual
output bf16(x + r)) must match bit for bit.  Results after a sum of squares
may differ from torch's reduction by an fp32 rounding of the mean, which can
move a bf16 output by one unit in the last place: those are checked to within
one bf16 ulp (2^-7 relative), with most elements equal.  SiLU uses the same
exp and division as torch's kernel.  The RoPE formula of the CPU path is
pinned separately by known answers (tests/test_qwen3_host.py).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

ULP = 2.0 ** -7


def _close(out, ref, min_equal=0.95):
    o, r = out.float(), ref.float()
    rel = ((o - r).abs() / r.abs().clamp_min(1e-30)).max().item()
    eq = (o == r).float().mean().item()
    assert rel <= ULP, f"max rel diff {rel:.3e}"
    assert eq >= min_equal, f"only {eq:.3f} of the elements equal"


def _rms_ref(x, w, eps, res=None):
    s = x.float() if res is None else x.float() + res.float()
    y = (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16) * w
    return y, s.to(torch.bfloat16)


@pytest.mark.parametrize("n,rows", [(2560, 7), (4096, 1), (8192, 3), (136, 2)])
def test_rmsnorm_with_and_without_residual(n, rows):
    from nanokv_amd.qwen3 import rmsnorm_dev

    g = torch.Generator(device="cuda").manual_seed(n + rows)
    x = (torch.randn(rows, n, generator=g, device="cuda") * 3).bfloat16()
    r = torch.randn(rows, n, generator=g, device="cuda").bfloat16()
    w = (1 + 0.1 * torch.randn(n, generator=g, device="cuda")).bfloat16()
    ref, _ = _rms_ref(x, w, 1e-6)
    _close(rmsnorm_dev(x, w, 1e-6), ref)
    out, res = rmsnorm_dev(x, w, 1e-6, r)
    ref, ref_res = _rms_ref(x, w, 1e-6, r)
    assert torch.equal(res, ref_res)
    _close(out, ref)


def test_qk_norm_rope_and_v_copy():
    from nanokv_amd.qwen3 import _rope_table, qk_norm_rope_dev

    T, hq, hkv, D, P = 9, 32, 8, 128, 4096
    g = torch.Generator(device="cuda").manual_seed(1)
    qkv = torch.randn(T, (hq + 2 * hkv) * D, generator=g, device="cuda").bfloat16()
    qw = (1 + 0.1 * torch.randn(D, generator=g, device="cuda")).bfloat16()
    kw = (1 + 0.1 * torch.randn(D, generator=g, device="cuda")).bfloat16()
    pos = torch.tensor([0, 1, 2, 63, 64, 1000, 4095, 17, 3000], device="cuda")
    cos, sin = _rope_table(D, 1e6, P, "cuda")
    q, k, v = qk_norm_rope_dev(qkv, pos, hq, hkv, qw, kw, 1e-6, cos, sin)

    def ref(x, w):
        xf = x.float()
        y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * w
        c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
        a, b = y.float().chunk(2, dim=-1)
        return torch.cat((a * c - b * s, b * c + a * s), dim=-1).to(torch.bfloat16)

    x = qkv.view(T, hq + 2 * hkv, D)
    _close(q, ref(x[:, :hq], qw))
    _close(k, ref(x[:, hq:hq + hkv], kw))
    assert torch.equal(v, x[:, hq + hkv:])
    assert q.is_contiguous() and k.is_contiguous() and v.is_contiguous()


def test_silu_mul_matches_torch():
    from nanokv_amd.qwen3 import silu_mul_dev

    g = torch.Generator(device="cuda").manual_seed(2)
    gu = (torch.randn(5, 2 * 9728, generator=g, device="cuda") * 4).bfloat16()
    ref = torch.nn.functional.silu(gu[:, :9728]) * gu[:, 9728:]
    _close(silu_mul_dev(gu), ref, min_equal=0.999)


@pytest.mark.parametrize("m,n,k", [(1, 6144, 2560), (1, 2560, 9728), (3, 1001, 4096), (4, 19456, 2560), (1, 7, 8)])
def test_gemv_against_float64(m, n, k):
    """|y - x.W^T| <= 2^-8 |x.W^T| (bf16 output rounding) + 2^-22 sum |x||W|
    (fp32 accumulation over at most 16384 terms, generous)."""
    from nanokv_amd.qwen3 import gemv_dev

    g = torch.Generator(device="cuda").manual_seed(m * n + k)
    x = torch.randn(m, k, generator=g, device="cuda").bfloat16()
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).bfloat16()
    y = gemv_dev(x, w).double()
    ref = x.double() @ w.double().T
    mag = x.double().abs() @ w.double().abs().T
    err = (y - ref).abs()
    bound = 2.0 ** -8 * ref.abs() + 2.0 ** -22 * mag + 1e-30
    assert bool((err <= bound).all()), f"worst err / bound {float((err / bound).max()):.3f}"


@pytest.mark.parametrize("m", [1, 2, 4])
def test_gemv_silu_mul_equals_gemv_then_silu_mul(m):
    """The fused gate|up projection + SiLU-and-mul rounds where the two
    launches do, so it matches them bit for bit."""
    from nanokv_amd.qwen3 import gemv_dev, gemv_silu_mul_dev, silu_mul_dev

    g = torch.Generator(device="cuda").manual_seed(31 + m)
    inter, k = 9728, 2560
    x = torch.randn(m, k, generator=g, device="cuda").bfloat16()
    w = (torch.randn(2 * inter, k, generator=g, device="cuda") * 0.05).bfloat16()
    assert torch.equal(gemv_silu_mul_dev(x, w), silu_mul_dev(gemv_dev(x, w)))
    # an odd intermediate size (the last row pair is half empty) against torch's SiLU
    w2 = w[: 2 * 1001].contiguous()
    gate, up = gemv_dev(x, w2[:1001]), gemv_dev(x, w2[1001:])
    _close(gemv_silu_mul_dev(x, w2), torch.nn.functional.silu(gate) * up, min_equal=0.99)
