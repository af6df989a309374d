"""GPU parity: causal conv1d (+SiLU, caches, varlen), L2 norm and gated RMSNorm vs the CPU oracle."""
import pytest
import torch

from oracle import (
    causal_conv1d_silu,
    causal_conv1d_varlen,
    conv_state_from_sequence,
    doc_ids_from_cu_seqlens,
    l2norm as l2norm_ref,
    rms_norm_gated as rms_norm_gated_ref,
)
from sorernn_amd import causal_conv1d, l2norm, rms_norm_gated
from sorernn_amd.ops import qkv_causal_conv1d
from tests.parity import assert_output_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("cu", [None, [0, 1, 3, 4, 70, 200, 300]], ids=["rows", "varlen"])
def test_conv_matches_oracle(dtype, cu):
    gen = torch.Generator().manual_seed(1)
    b = 2 if cu is None else 1
    x = torch.randn(b, 300, 384, generator=gen).to(dtype)
    w = torch.randn(384, 4, generator=gen) * 0.5
    cu_t = None if cu is None else torch.tensor(cu)
    y, fin = causal_conv1d(x.to(DEV), w.to(DEV), activation="silu", output_final_state=True,
                           cu_seqlens=None if cu_t is None else cu_t.to(DEV), cu_seqlens_cpu=cu_t)
    y_ref = causal_conv1d_silu(x, w, cu_t)
    assert_output_close(y.cpu(), y_ref, tol=1e-2 if dtype == torch.bfloat16 else 1e-5)
    assert torch.equal(fin.cpu(), conv_state_from_sequence(x, 4, cu_t))


def test_conv_tap_order_and_no_activation():
    x = torch.zeros(1, 5, 64)
    x[0, 2, :] = 1.0
    w = torch.zeros(64, 3)
    w[:, 0], w[:, 1], w[:, 2] = 1.0, 10.0, 100.0
    y, _ = causal_conv1d(x.to(DEV), w.to(DEV), activation=None)
    assert y[0, :, 0].cpu().tolist() == [0.0, 0.0, 100.0, 10.0, 1.0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_initial_state_continues_sequence(dtype):
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(2, 50, 128, generator=gen).to(dtype)
    w = torch.randn(128, 4, generator=gen)
    full, _ = causal_conv1d(x.to(DEV), w.to(DEV), activation="silu")
    _, cache = causal_conv1d(x[:, :20].to(DEV), w.to(DEV), activation="silu", output_final_state=True)
    tail, _ = causal_conv1d(x[:, 20:].contiguous().to(DEV), w.to(DEV), activation="silu", initial_state=cache)
    # the same fp32 sums of the same inputs: bit-identical
    assert torch.equal(tail.cpu(), full[:, 20:].cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_varlen_initial_states_match_oracle(dtype):
    """Per-document initial conv caches (documents of 1, 2, 1, 66 and 30 tokens; the 16-bit path
    walks 32-token blocks, so documents start inside and at the edges of blocks)."""
    gen = torch.Generator().manual_seed(4)
    bounds = [0, 1, 3, 4, 70, 100]
    t, c, wd = bounds[-1], 256, 4
    x = torch.randn(1, t, c, generator=gen).to(dtype)
    init = torch.randn(len(bounds) - 1, c, wd, generator=gen).to(dtype)
    w = torch.randn(c, wd, generator=gen) * 0.5
    cu = torch.tensor(bounds)
    y, fin = causal_conv1d(x.to(DEV), w.to(DEV), activation="silu", initial_state=init.to(DEV),
                           output_final_state=True, cu_seqlens=cu.to(DEV), cu_seqlens_cpu=cu)
    for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        # the cache's last W-1 inputs (newest last) precede the document
        seq = torch.cat([init[n, :, 1:].T[None], x[:, a:e]], dim=1)
        ref = causal_conv1d_silu(seq, w, None)[:, wd - 1:]
        assert_output_close(y[:, a:e].cpu(), ref, tol=1e-2 if dtype == torch.bfloat16 else 1e-5)
        assert torch.equal(fin[n].cpu(), seq[0, -wd:].T)


def test_conv_nan_does_not_leak_across_documents():
    cu = torch.tensor([0, 4, 9])
    x = torch.randn(1, 9, 64)
    x[:, 3] = float("nan")
    y, _ = causal_conv1d(x.to(DEV), torch.randn(64, 4).to(DEV), cu_seqlens=cu.to(DEV), cu_seqlens_cpu=cu)
    y = y.cpu()
    assert torch.isfinite(y[:, 4:]).all() and torch.isnan(y[:, 3]).all()
    ids = doc_ids_from_cu_seqlens(cu, 9)
    ref = causal_conv1d_varlen(x.double(), torch.zeros(64, 4, dtype=torch.float64), ids)
    assert ref.shape == y.shape


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_l2norm_matches_oracle(dtype):
    x = (torch.randn(37, 3, 128) * 4).to(dtype)
    x[0, 0] = 0
    y = l2norm(x.to(DEV)).cpu()
    assert_output_close(y, l2norm_ref(x), tol=1e-2 if dtype == torch.bfloat16 else 1e-6)
    assert (y[0, 0] == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128])
def test_rms_norm_gated_matches_oracle(dtype, d):
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(4, 33, 16, d, generator=gen).to(dtype)
    gate = torch.randn(4, 33, 16, d, generator=gen).to(dtype)
    w = torch.randn(d, generator=gen)
    y = rms_norm_gated(x.to(DEV), gate.to(DEV), w.to(DEV), None, activation="swish", eps=1e-6).cpu()
    assert_output_close(y, rms_norm_gated_ref(x, gate, w, 1e-6), tol=2e-2 if dtype == torch.bfloat16 else 1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("cu", [None, [0, 1, 3, 40, 41, 200]], ids=["rows", "varlen"])
def test_qkv_conv_equals_three_convs_and_l2norm(dtype, head_dim, cu):
    """The fused prologue (one launch over q | k | v read from a wider projection row) equals three
    causal_conv1d calls followed by l2norm of every q/k head up to fp32 rounding: the conv and SiLU
    are the same formulas (the kernels may contract a multiply-add differently), and the norm is
    v_rsq_f32 of max(|x|^2, 1e-24) against the row kernel's 1 / max(sqrt(|x|^2), 1e-12). So the
    outputs are within two ulps and almost always equal."""
    gen = torch.Generator().manual_seed(5)
    b = 2 if cu is None else 1
    t, cqk, cv = 200, 2 * head_dim, 4 * head_dim
    proj = torch.randn(b, t, 2 * cqk + cv + 64, generator=gen).to(dtype).to(DEV)  # 64 extra columns per row
    w = (torch.randn(2 * cqk + cv, 4, generator=gen) * 0.5).to(DEV)
    cu_t = None if cu is None else torch.tensor(cu)
    kw = dict(cu_seqlens=None if cu_t is None else cu_t.to(DEV), cu_seqlens_cpu=cu_t)
    q, k, v = qkv_causal_conv1d(proj, w, cqk, cv, head_dim, **kw)
    parts = (proj[..., :cqk], proj[..., cqk:2 * cqk], proj[..., 2 * cqk:2 * cqk + cv])
    wq, wk, wv = w[:cqk], w[cqk:2 * cqk], w[2 * cqk:]
    rq = causal_conv1d(parts[0].contiguous(), wq, activation="silu", **kw)[0]
    rk = causal_conv1d(parts[1].contiguous(), wk, activation="silu", **kw)[0]
    rv = causal_conv1d(parts[2].contiguous(), wv, activation="silu", **kw)[0]
    rq = l2norm(rq.view(b, t, -1, head_dim)).view(b, t, cqk)
    rk = l2norm(rk.view(b, t, -1, head_dim)).view(b, t, cqk)
    # one ulp of x is at most |x| 2^-7 (bf16) or |x| 2^-10 (fp16); q/k are rounded twice (conv, norm)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    for out, ref, nm in ((q, rq, "q"), (k, rk, "k"), (v, rv, "v")):
        o, r = out.float(), ref.float()
        assert ((o - r).abs() <= 2 * ulp * r.abs().clamp_min(2.0 ** -14)).all(), f"{nm}: more than two ulps apart"
        assert (out != ref).float().mean().item() <= 1e-2, f"{nm}: {(out != ref).float().mean().item():.2%} differ"
