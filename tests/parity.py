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


# Gradients: the reference's own bar for FLA against autograd through its torch path
# (tests/model/test_gdn.py:98-101,156-162): rtol 1e-2 and atol 5e-3 * max|ref| (5e-2 for the
# per-head sums A_log and dt_bias).
GRAD_RTOL = 1e-2
GRAD_ATOL_FRAC = 5e-3


def assert_grad_close(out: torch.Tensor, ref: torch.Tensor, what: str, atol_frac: float = GRAD_ATOL_FRAC) -> float:
    """Assert ``|out - ref| <= atol_frac * max|ref| + GRAD_RTOL * |ref|`` elementwise; return max-err / max|ref|."""
    assert out is not None, f"{what}: no gradient"
    assert out.shape == ref.shape, f"{what}: shape {tuple(out.shape)} != {tuple(ref.shape)}"
    o, r = out.detach().double().cpu(), ref.detach().double().cpu()
    assert torch.isfinite(o).all(), f"{what}: non-finite values"
    scale = float(r.abs().max()) if r.numel() else 0.0
    err = (o - r).abs()
    bound = atol_frac * scale + GRAD_RTOL * r.abs()
    bad = err > bound
    rel = float(err.max()) / scale if scale > 0 else float(err.max()) if err.numel() else 0.0
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.numel()} elements outside tolerance; "
                           f"max err {float(err.max()):.3e}, max|ref| {scale:.3e}")
    return rel
