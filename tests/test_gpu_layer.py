"""GPU: the GatedDeltaNet layer on the gfx950 ops (``sorernn_amd.gdn_layer``) vs the oracle composition.

Mirrors the reference's layer tests (``tests/model/test_gdn.py``): parity of the kernel path with
the pure-torch path on shared weights (there FLA vs torch, ``:74-101,128-162``), packed == separate
(``:41-48``), batch rows are independent documents (``:51-57``), document isolation with a negative
control (``:165-193``), and the no-host-sync property of the packed path (``tests/model/test_lm.py:292-321``).
"""
import pytest
import torch

import torch.nn.functional as F

from oracle import causal_conv1d_silu, gate_and_beta, l2norm, recurrent_gated_delta_rule, rms_norm, rms_norm_gated
from sorernn_amd.gdn_layer import GatedDeltaNet, GDNLayerConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16


def _layer(kernel_gate=True, rep=2, seed=0, d_model=256, head_dim=128, fla_conv=True, fused_norm_gate=True):
    """The layer with the caller flags of the reference's training presets (gdn_fla_conv and
    fused_norm_gate on, sore/model/config.py:116,123) unless asked otherwise."""
    torch.manual_seed(seed)
    cfg = GDNLayerConfig(d_model=d_model, gdn_qk_heads=2, gdn_v_heads=2 * rep, gdn_head_dim=head_dim,
                         gdn_kernel_gate=kernel_gate, gdn_fla_conv=fla_conv, fused_norm_gate=fused_norm_gate)
    return GatedDeltaNet(cfg)


def _oracle_forward(layer, x, cu=None):
    """The same layer computed with the CPU oracle in fp32 (bf16 rounding where the GPU path stores bf16),
    with the rounding points of the layer's caller flags: without gdn_fla_conv the conv weight is
    rounded to bf16 and the conv output rounded before the SiLU (sore/model/gdn.py:208-209); without
    fused_norm_gate RMSNorm(o) is rounded to bf16 before the product with silu(gate) (gdn.py:188)."""
    b, t, _ = x.shape
    hd, hq, hv = layer.head_dim, layer.qk_heads, layer.v_heads
    with torch.no_grad():
        xb = x.to(BF16).float()
        lin = lambda m: (xb @ m.weight.to(BF16).float().T).to(BF16)  # noqa: E731  bf16 GEMM, bf16 output

        def conv(h, w):
            if layer.fla_conv:
                return causal_conv1d_silu(h, w.float(), cu)
            return F.silu(causal_conv1d_silu(h, w.to(BF16).float(), cu, activation=None).float()).to(BF16)

        q = conv(lin(layer.q_proj), layer.conv_q).view(b, t, hq, hd)
        k = conv(lin(layer.k_proj), layer.conv_k).view(b, t, hq, hd)
        v = conv(lin(layer.v_proj), layer.conv_v).view(b, t, hv, hd)
        g, beta = gate_and_beta(lin(layer.a_proj), lin(layer.b_proj), layer.A_log, layer.dt_bias)
        o, _ = recurrent_gated_delta_rule(l2norm(q), l2norm(k), v, g, beta, hd**-0.5, cu_seqlens=cu)
        gate = lin(layer.g_proj).view(b, t, hv, hd)
        if layer.fused_norm_gate:
            o = rms_norm_gated(o, gate, layer.o_norm.weight, layer.o_norm.eps)
        else:
            o = (rms_norm(o, layer.o_norm.weight, layer.o_norm.eps).float() * F.silu(gate.float()).to(BF16).float())
            o = o.to(BF16)
        return o.flatten(-2).float() @ layer.o_proj.weight.to(BF16).float().T


def _run(layer, x, cu=None):
    cu_dev = None if cu is None else cu.to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
        return layer(x.to(DEV), cu_seqlens=cu_dev, cu_seqlens_cpu=cu).float().cpu()


# the reference's options matrix (tests/model/test_gdn.py:104-162): GVA 1 and 2, documents of 1-3
# tokens and one document over the whole window, plus plain batch rows
_CU_CASES = {"rows": None, "short_docs": [0, 1, 3, 4, 70, 200, 512], "one_doc": [0, 512]}


@pytest.mark.parametrize("kernel_gate", [True, False], ids=["kernel_gate", "torch_gate"])
@pytest.mark.parametrize("cu_case", sorted(_CU_CASES))
@pytest.mark.parametrize("rep", [1, 2], ids=["no_gva", "gva2x"])
def test_layer_matches_oracle(kernel_gate, cu_case, rep):
    cu = _CU_CASES[cu_case]
    layer = _layer(kernel_gate, rep=rep)
    b = 2 if cu is None else 1
    x = torch.randn(b, 512, 256, generator=torch.Generator().manual_seed(2))
    cu_t = None if cu is None else torch.tensor(cu)
    ref = _oracle_forward(layer, x, cu_t)
    out = _run(layer.to(DEV), x, cu_t)
    err = (out - ref).abs().max().item()
    assert err <= 2e-2 * ref.abs().max().item() + 1e-3, f"max-abs error {err:.3e} (max|ref| {ref.abs().max():.3e})"


@pytest.mark.parametrize("route", ["inference", "reference"])
@pytest.mark.parametrize("cu_case", ["rows", "short_docs"])
def test_layer_unfused_caller_flags_match_oracle(route, cu_case):
    """gdn_fla_conv and fused_norm_gate off (the reference's ModelConfig defaults): the layer takes the
    reference's rounding points (conv weight in bf16 and the conv output rounded before F.silu,
    o_norm(o) rounded before the gate product), on both of its routes."""
    cu = _CU_CASES[cu_case]
    layer = _layer(True, rep=2, fla_conv=False, fused_norm_gate=False)
    b = 2 if cu is None else 1
    x = torch.randn(b, 512, 256, generator=torch.Generator().manual_seed(12))
    cu_t = None if cu is None else torch.tensor(cu)
    ref = _oracle_forward(layer, x, cu_t)
    layer = layer.to(DEV)
    if route == "inference":
        out = _run(layer, x, cu_t)
    else:
        with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
            cu_dev = None if cu_t is None else cu_t.to(DEV)
            out = layer._forward_reference(x.to(DEV), cu_seqlens=cu_dev, cu_seqlens_cpu=cu_t).float().cpu()
    err = (out - ref).abs().max().item()
    assert err <= 2e-2 * ref.abs().max().item() + 1e-3, f"max-abs error {err:.3e} (max|ref| {ref.abs().max():.3e})"
    # negative control: the fused-flag oracle differs from the unfused one at these rounding points
    layer.fla_conv = layer.fused_norm_gate = True
    assert (_oracle_forward(layer.cpu(), x, cu_t) - ref).abs().max() > 0


def test_layer_packed_equals_separate_and_no_host_sync():
    layer = _layer().to(DEV)
    x = torch.randn(1, 300, 256, generator=torch.Generator().manual_seed(3))
    cu = torch.tensor([0, 70, 300])
    cu_dev = cu.to(DEV)
    xd = x.to(DEV)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")  # any device->host sync in the packed forward raises
    try:
        with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
            packed = layer(xd, cu_seqlens=cu_dev, cu_seqlens_cpu=cu)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    packed = packed.float().cpu()
    sep = torch.cat([_run(layer, x[:, :70]), _run(layer, x[:, 70:])], dim=1)
    torch.testing.assert_close(packed, sep, atol=2e-2, rtol=0)
    # negative control: without cu_seqlens the second document sees the first one's state and conv
    whole = _run(layer, x)
    assert (whole[:, 70:] - sep[:, 70:]).abs().max() > 1e-2


def test_layer_batch_rows_are_independent_documents():
    layer = _layer().to(DEV)
    x = torch.randn(3, 90, 256, generator=torch.Generator().manual_seed(4))
    batched = _run(layer, x)
    rows = torch.cat([_run(layer, x[i : i + 1]) for i in range(3)], dim=0)
    torch.testing.assert_close(batched, rows, atol=2e-2, rtol=0)


def test_layer_documents_are_isolated():
    layer = _layer().to(DEV)
    cu = torch.tensor([0, 1, 3, 4, 70, 200, 512])
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(1, 512, 256, generator=gen)
    out = _run(layer, x, cu)
    for start, end in ((0, 4), (4, 70)):
        x2 = x.clone()
        x2[:, start:end] = torch.randn(1, end - start, 256, generator=gen)
        out2 = _run(layer, x2, cu)
        assert torch.equal(out[:, end:], out2[:, end:]), f"documents after [{start},{end}) changed"
        assert not torch.allclose(out[:, start:end], out2[:, start:end], atol=1e-3)
        leak, leak2 = _run(layer, x), _run(layer, x2)  # negative control without cu_seqlens
        assert (leak[:, end:] - leak2[:, end:]).abs().max() > 1e-3


def test_layer_state_dict_names_match_reference():
    names = set(_layer().state_dict())
    expected = {"q_proj.weight", "k_proj.weight", "v_proj.weight", "g_proj.weight", "a_proj.weight", "b_proj.weight",
                "conv_q", "conv_k", "conv_v", "A_log", "dt_bias", "o_norm.weight", "o_proj.weight"}
    assert names == expected


@pytest.mark.parametrize("kernel_gate", [True, False], ids=["kernel_gate", "torch_gate"])
@pytest.mark.parametrize("cu", [None, [0, 1, 3, 4, 70, 200, 512]], ids=["rows", "short_docs"])
def test_inference_route_matches_reference_route(kernel_gate, cu):
    """With autograd off the layer fuses its projections and its q/k/v prologue; the output equals
    the reference-expression route up to the GEMMs' accumulation order."""
    layer = _layer(kernel_gate).to(DEV)
    b = 2 if cu is None else 1
    x = torch.randn(b, 512, 256, generator=torch.Generator().manual_seed(3)).to(DEV)
    cu_t = None if cu is None else torch.tensor(cu)
    cu_dev = None if cu_t is None else cu_t.to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
        fused = layer(x, cu_seqlens=cu_dev, cu_seqlens_cpu=cu_t).float()
        ref = layer._forward_reference(x, cu_seqlens=cu_dev, cu_seqlens_cpu=cu_t).float()
    rel = ((fused - ref).norm() / ref.norm()).item()
    assert rel <= 1e-2, f"relative L2 {rel:.3e}"


def test_layer_extreme_inputs_stay_finite():
    """x100 inputs (reference tests/model/test_gdn.py:60-71) through the bf16 layer: output and input
    gradient finite, with packed documents, and the chunk kernel's fp16 operands inside their range
    (the range guard's flag stays clear)."""
    import sorernn_amd

    sorernn_amd.check_chunk_range()
    torch.manual_seed(0)
    cfg = GDNLayerConfig(d_model=128, gdn_qk_heads=2, gdn_v_heads=4, gdn_head_dim=64, gdn_kernel_gate=True,
                         gdn_fla_conv=True, fused_norm_gate=True)
    layer = GatedDeltaNet(cfg).to(DEV)
    x = (torch.randn(1, 64, 128, generator=torch.Generator().manual_seed(6)) * 100).to(DEV).requires_grad_(True)
    cu = torch.tensor([0, 30, 64])
    with torch.autocast("cuda", dtype=BF16):
        out = layer(x, cu_seqlens=cu.to(DEV), cu_seqlens_cpu=cu)
    assert torch.isfinite(out).all()
    out.float().square().mean().backward()
    torch.cuda.synchronize()
    assert torch.isfinite(x.grad).all()
    assert not sorernn_amd.check_chunk_range(), "x100 layer inputs overflowed the chunk kernel's fp16 operands"


def test_layer_cu_seqlens_cpu_is_exact():
    """cu_seqlens_cpu only saves reading cu_seqlens back on the host: the same values reach the same
    kernels, so output and gradients are bitwise equal with and without it (reference
    tests/model/test_lm.py:339-361); two runs without it are first shown bitwise equal."""
    cu = torch.tensor([0, 1, 3, 4, 70, 200, 300])
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(1, 300, 128, generator=gen)
    cot = torch.randn(1, 300, 128, generator=gen)

    def run(with_cpu):
        torch.manual_seed(0)
        cfg = GDNLayerConfig(d_model=128, gdn_qk_heads=2, gdn_v_heads=4, gdn_head_dim=64, gdn_kernel_gate=True,
                         gdn_fla_conv=True, fused_norm_gate=True)
        layer = GatedDeltaNet(cfg).to(DEV)
        xd = x.to(DEV).requires_grad_(True)
        with torch.autocast("cuda", dtype=BF16):
            out = layer(xd, cu_seqlens=cu.to(DEV), cu_seqlens_cpu=cu if with_cpu else None)
        (out.float() * cot.to(DEV)).sum().backward()
        torch.cuda.synchronize()
        return out.detach(), xd.grad, {n: p.grad for n, p in layer.named_parameters()}

    a, b, c = run(False), run(False), run(True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and all(torch.equal(a[2][n], b[2][n]) for n in a[2]), \
        "two identical runs differ: the bitwise comparison below would prove nothing"
    assert torch.equal(c[0], a[0]) and torch.equal(c[1], a[1])
    for n in a[2]:
        assert torch.equal(c[2][n], a[2][n]), n
