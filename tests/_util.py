"""Small helpers shared by the tests (conversions between torch and the oracle)."""

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    """bf16 / fp32 torch tensor -> float32 numpy array (exact for bf16)."""
    return t.detach().to("cpu", torch.float32).numpy()


def bf16(a) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)


def f32_bits(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32)


def assert_close_bf16(out, ref, *, rel=2.0 ** -7, abs_tol=2e-5, bar=2e-3):
    """Kernel output (bf16) vs fp64 oracle: within ~1 bf16 ulp, and under the 2e-3 bar."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(out - ref)
    assert np.isfinite(out).all(), "non-finite kernel output"
    worst = float(err.max())
    assert worst <= bar, f"max |err| {worst:.3e} exceeds {bar}"
    bad = err > rel * np.abs(ref) + abs_tol
    assert not bad.any(), (
        f"{int(bad.sum())} of {bad.size} outputs off by more than rel {rel} + abs {abs_tol}: "
        f"worst {worst:.3e}")
    return worst


# The matrix-core (prefill) kernel rounds the softmax probabilities to bf16 for
# the P.V product, as the reference's flash-attention prefill does.  With few
# keys and nearly uniform probabilities that rounding alone moves an output by
# up to ~1.1e-4 (a CPU emulation of bf16 P reproduces the kernel's worst
# error exactly), so its outputs get this absolute slack; the 2e-3 bar holds.
PREFILL_TOL = dict(rel=2.0 ** -7, abs_tol=2e-4)
