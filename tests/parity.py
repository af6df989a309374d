"""Tolerances of the GDN path and helpers to assert them.

- outputs: max-abs error <= 2e-2 for bf16 outputs (fp32 outputs use 2e-3);
- final states (fp32): relative L2 error <= 1e-3.
"""
import torch

OUT_MAXABS = {torch.bfloat16: 2e-2, torch.float16: 1e-2, torch.float32: 2e-3}
STATE_REL_L2 = 1e-3


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max()) if a.numel() else 0.0


def assert_output_close(out: torch.Tensor, ref: torch.Tensor, tol: float | None = None, what: str = "o") -> float:
    assert out.shape == ref.shape, f"{what}: shape {tuple(out.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(out).all(), f"{what}: non-finite values"
    err = max_abs(out, ref)
    tol = OUT_MAXABS[out.dtype] if tol is None else tol
    assert err <= tol, f"{what}: max-abs error {err:.3e} > {tol:.1e}"
    return err


def assert_state_close(st: torch.Tensor, ref: torch.Tensor, tol: float = STATE_REL_L2, what: str = "final_state") -> float:
    assert st.shape == ref.shape, f"{what}: shape {tuple(st.shape)} != {tuple(ref.shape)}"
    assert st.dtype == torch.float32
    assert torch.isfinite(st).all(), f"{what}: non-finite values"
    err = rel_l2(st, ref)
    assert err <= tol, f"{what}: relative L2 error {err:.3e} > {tol:.1e}"
    return err
