"""GPU parity of the chunked prefill's T-solve kernel (``gated_delta_chunk_prep_kernel``) on its own.

``gdn_chunk_fwd`` leaves the per-chunk rows of T - I = (I + A)^-1 - I in its workspace (fp16
``[tokens][HV][64]``, columns in the state kernel's contraction order: token j of the chunk at column
32(j // 32) + 8((j // 4) % 4) + 4((j // 16) % 2) + j % 4). This test reads them back and compares
them with T computed in fp64 on the CPU from the same k, g and beta: A_tj = beta_t exp(gam_t - gam_j)
k_t.k_j for j < t within a chunk (gam = in-chunk cumsum of g; sore/model/gdn_ref.py:17-21 in chunk
form, oracle/gdn_oracle.py::_chunk_segment). Bar: the fp16 rounding of T plus fp32 accumulation,
max |err| <= 4e-3 * max(1, max|T|) per chunk. Rows past a sequence's end are not written.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from sorernn_amd import _lib
from sorernn_amd.ops import chunk_workspace_bytes
from sorernn_amd.synthetic import gdn_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"
C = 64


def _tok_col(j: np.ndarray) -> np.ndarray:
    return (j & ~31) + 8 * ((j >> 2) & 3) + 4 * ((j >> 4) & 1) + (j & 3)


def _run(inp, flags=0, a_log=None, dt_bias=None):
    """gdn_chunk_fwd on the GPU; returns the workspace's T - I rows as fp64 [tokens, HV, 64] in
    natural token order."""
    d = inp.to(DEV)
    b, t, h, kd = inp.q.shape
    hv, vd = inp.v.shape[2], inp.v.shape[3]
    cu = d.cu_seqlens
    n = b if cu is None else cu.numel() - 1
    o = torch.empty(b, t, hv, vd, device=DEV, dtype=torch.bfloat16)
    nbytes = chunk_workspace_bytes(b, t, hv, n, cu is not None)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    _lib.call("gdn_chunk_fwd", _lib.ptr(d.q), _lib.ptr(d.k), _lib.ptr(d.v), _lib.ptr(d.g), _lib.ptr(d.beta), None,
              _lib.ptr(o), None, _lib.ptr(cu), b, t, h, hv, kd, vd, n, _lib.DTYPE_BF16, _lib.dtype_code(d.g.dtype),
              _lib.dtype_code(d.beta.dtype), inp.scale, flags, _lib.ptr(a_log), _lib.ptr(dt_bias), _lib.ptr(ws),
              nbytes, _lib.stream_of(d.q))
    torch.cuda.synchronize()
    rows = ws[: b * t * hv * C * 2].view(torch.float16).view(b * t, hv, C).cpu().double().numpy()
    nat = np.empty_like(rows)
    nat[:, :, :] = rows[:, :, _tok_col(np.arange(C))]
    return nat


def _ref_rows(inp, flags=0, a_log=None, dt_bias=None):
    """fp64 T - I rows [tokens, HV, 64] (natural column order) and the chunk spans."""
    b, t, h, kd = inp.q.shape
    hv = inp.v.shape[2]
    rep = hv // h
    k = inp.k.float()
    if flags & _lib.FLAG_QK_L2NORM:
        k = F.normalize(k, dim=-1).to(torch.bfloat16).float()
    k = k.double().reshape(b * t, h, kd)
    g = inp.g.double().reshape(b * t, hv)
    beta = inp.beta.double().reshape(b * t, hv)
    if flags & _lib.FLAG_GATE_IN_KERNEL:
        g = -a_log.cpu().double().exp() * F.softplus(g + dt_bias.cpu().double())
    if flags & _lib.FLAG_BETA_SIGMOID:
        beta = beta.sigmoid()
    if inp.cu_seqlens is None:
        bounds = [(i * t, (i + 1) * t) for i in range(b)]
    else:
        cu = inp.cu_seqlens.tolist()
        bounds = list(zip(cu[:-1], cu[1:]))
    out = np.zeros((b * t, hv, C))
    spans = []
    for bos, eos in bounds:
        for c0 in range(bos, eos, C):
            ln = min(C, eos - c0)
            spans.append((c0, ln))
            for j in range(hv):
                kk = k[c0:c0 + ln, j // rep]
                gam = g[c0:c0 + ln, j].cumsum(0)
                a = beta[c0:c0 + ln, j, None] * (gam[:, None] - gam[None, :]).exp() * (kk @ kk.T)
                a = torch.tril(a, -1)
                tm = torch.linalg.inv(torch.eye(ln, dtype=torch.float64) + a) - torch.eye(ln, dtype=torch.float64)
                out[c0:c0 + ln, j, :ln] = tm.numpy()
    return out, spans


def _check(inp, **kw):
    got = _run(inp, **kw)
    ref, spans = _ref_rows(inp, **kw)
    worst = 0.0
    for c0, ln in spans:
        g_, r_ = got[c0:c0 + ln], ref[c0:c0 + ln]
        err = np.abs(g_ - r_).max() / max(1.0, np.abs(r_).max())
        worst = max(worst, err)
        assert np.isfinite(g_).all()
        assert err <= 4e-3, f"chunk at token {c0} (len {ln}): max err {err:.3e}"
    return worst


@pytest.mark.parametrize("kd", [128, 64], ids=lambda k: f"K{k}")
@pytest.mark.parametrize("t", [256, 200, 37], ids=lambda t: f"T{t}")
def test_tsolve_fixed_length(kd, t):
    print(f"tsolve K={kd} T={t}", flush=True)
    _check(gdn_inputs(2, t, 3, kd, dtype=torch.bfloat16, seed=11 + t))


@pytest.mark.parametrize("rep", [1, 2], ids=["no_gva", "gva2x"])
def test_tsolve_varlen(rep):
    print(f"tsolve varlen rep={rep}", flush=True)
    cu = torch.tensor([0, 1, 3, 64, 65, 200, 329, 512])
    _check(gdn_inputs(1, 512, 2, 128, HV=2 * rep, dtype=torch.bfloat16, seed=3, cu_seqlens=cu))


def test_tsolve_in_kernel_gate_sigmoid_l2norm():
    print("tsolve in-kernel gate, beta sigmoid, k L2 norm", flush=True)
    inp = gdn_inputs(1, 192, 2, 128, HV=4, dtype=torch.bfloat16, seed=5)
    gen = torch.Generator().manual_seed(6)
    inp.k = (3.0 * torch.randn(inp.k.shape, generator=gen)).to(torch.bfloat16)  # not unit norm
    inp.g = torch.randn(inp.g.shape, generator=gen)      # raw gate logits a
    inp.beta = torch.randn(inp.beta.shape, generator=gen)  # raw beta logits b
    a_log = torch.rand(4, generator=gen) * 2
    dt_bias = torch.randn(4, generator=gen) * 0.5
    flags = _lib.FLAG_QK_L2NORM | _lib.FLAG_GATE_IN_KERNEL | _lib.FLAG_BETA_SIGMOID
    _check(inp, flags=flags, a_log=a_log.to(DEV), dt_bias=dt_bias.to(DEV))
