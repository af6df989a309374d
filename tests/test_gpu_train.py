"""GPU: backward of the prologue/epilogue operators and of the whole GatedDeltaNet layer.

- ``causal_conv1d`` (+ SiLU, bias, per-document reset, initial conv state), ``l2norm`` and
  ``rms_norm_gated`` against fp64 autograd through the oracle functions (the reference's own conv
  gradient tests compare against ``F.conv1d`` autograd, ``tests/model/test_conv.py:66-91``), with
  the reference's gradient tolerance (``tests/parity.py::assert_grad_close``).
- The layer: every parameter's gradient and the input gradient of the bf16 layer on the gfx950 ops
  against fp64 autograd through the oracle composition on the same weights (the reference's
  ``test_fla_options_match_torch_backend``, ``tests/model/test_gdn.py:128-162``). The layer runs in
  bf16 end to end here (the chunk kernels take bf16 q/k/v), so this check is a relative L2 error
  of 3e-2 per tensor: wiring mistakes (a missing gradient, a wrong sign or scale) are O(1).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import causal_conv1d_varlen, doc_ids_from_cu_seqlens, recurrent_gated_delta_rule
from sorernn_amd import causal_conv1d, l2norm, rms_norm_gated
from sorernn_amd.gdn_layer import GatedDeltaNet, GDNLayerConfig
from tests.parity import assert_grad_close, rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _conv_ref(x, w, bias, init, cu, act):
    """fp64 conv with an initial conv state: document n is preceded by init[n, :, 1:] (oldest first)."""
    t = x.shape[1]
    bounds = [0, t] if cu is None else [int(v) for v in cu.tolist()]
    outs = []
    for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        xs = x[:, a:e]
        pre = init[n, :, 1:].T[None] if init is not None else torch.zeros(1, w.shape[1] - 1, x.shape[2], dtype=x.dtype)
        y = causal_conv1d_varlen(torch.cat([pre, xs], 1), w, None)[:, pre.shape[1]:]
        outs.append(y)
    y = torch.cat(outs, 1)
    if bias is not None:
        y = y + bias
    return F.silu(y) if act else y


@pytest.mark.parametrize("case", [
    dict(cu=None, act=True, bias=True, init=False, w=4),
    dict(cu=[0, 1, 3, 4, 70, 200, 300], act=True, bias=False, init=True, w=4),
    dict(cu=[0, 63, 64, 65, 129, 300], act=False, bias=True, init=True, w=3),
], ids=["plain", "short_docs_init", "chunk_edges"])
def test_causal_conv1d_backward(case):
    gen = torch.Generator().manual_seed(21)
    t, c, w = 300, 96, case["w"]
    cu = None if case["cu"] is None else torch.tensor(case["cu"])
    n = 1 if cu is None else len(case["cu"]) - 1
    x = torch.randn(1, t, c, generator=gen).to(torch.bfloat16)
    wt = torch.randn(c, w, generator=gen) * 0.5
    bias = torch.randn(c, generator=gen) if case["bias"] else None
    init = torch.randn(n, c, w, generator=gen).to(torch.bfloat16) if case["init"] else None
    dy = torch.randn(1, t, c, generator=gen).to(torch.bfloat16)
    leaves = [None if v is None else v.to(DEV).requires_grad_(True) for v in (x, wt, bias, init)]
    y, _ = causal_conv1d(leaves[0], leaves[1], leaves[2], initial_state=leaves[3], activation="silu" if case["act"] else None,
                         cu_seqlens=None if cu is None else cu.to(DEV), cu_seqlens_cpu=cu)
    y.backward(dy.to(DEV))
    refs = [None if v is None else v.double().requires_grad_(True) for v in (x, wt, bias, init)]
    yr = _conv_ref(refs[0], refs[1], refs[2], refs[3], cu, case["act"])
    yr.backward(dy.double())
    for name, a, r in zip(("dx", "dweight", "dbias", "dinit"), leaves, refs):
        if a is None:
            continue
        rel = assert_grad_close(a.grad, r.grad, name)
        print(f"  conv {name}: {rel:.2e}", flush=True)


def test_l2norm_backward():
    gen = torch.Generator().manual_seed(22)
    x = (torch.randn(333, 128, generator=gen) * 3).to(torch.bfloat16)
    x[5] = 0  # clamped row: the gradient is dy / eps there, as F.normalize's
    dy = torch.randn(333, 128, generator=gen).to(torch.bfloat16)
    xd = x.to(DEV).requires_grad_(True)
    l2norm(xd).backward(dy.to(DEV))
    xr = x.double().requires_grad_(True)
    F.normalize(xr, dim=-1).backward(dy.double())
    ok = torch.ones(333, dtype=torch.bool)
    ok[5] = False
    assert_grad_close(xd.grad[ok], xr.grad[ok], "dx")
    assert torch.isfinite(xd.grad).all()


@pytest.mark.parametrize("act", ["swish", None])
def test_rms_norm_gated_backward(act):
    gen = torch.Generator().manual_seed(23)
    x = torch.randn(2, 70, 4, 128, generator=gen).to(torch.bfloat16)
    g = torch.randn(2, 70, 4, 128, generator=gen).to(torch.bfloat16)
    wt = torch.randn(128, generator=gen)
    bias = torch.randn(128, generator=gen) * 0.1
    dy = torch.randn(2, 70, 4, 128, generator=gen).to(torch.bfloat16)
    leaves = [v.to(DEV).requires_grad_(True) for v in (x, g, wt, bias)]
    rms_norm_gated(*leaves, activation=act, eps=1e-6).backward(dy.to(DEV))
    xr, gr, wr, br = [v.double().requires_grad_(True) for v in (x, g, wt, bias)]
    n = xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6) * wr + br
    (n * (F.silu(gr) if act else gr)).backward(dy.double())
    for name, a, r in zip(("dx", "dgate", "dweight", "dbias"), leaves, (xr, gr, wr, br)):
        rel = assert_grad_close(a.grad, r.grad, name)
        print(f"  rms {name}: {rel:.2e}", flush=True)


def _oracle_layer_loss(layer, x, cotangent, cu):
    """fp64 autograd through the oracle composition of the layer on the layer's own (fp64) parameters."""
    p = {n: v.detach().double().requires_grad_(True) for n, v in layer.named_parameters()}
    b, t, _ = x.shape
    hd, hq, hv = layer.head_dim, layer.qk_heads, layer.v_heads
    xr = x.double().requires_grad_(True)
    ids = None if cu is None else doc_ids_from_cu_seqlens(cu, t)
    conv = lambda h, w: F.silu(causal_conv1d_varlen(h, w, ids))  # noqa: E731
    q = conv(xr @ p["q_proj.weight"].T, p["conv_q"]).view(b, t, hq, hd)
    k = conv(xr @ p["k_proj.weight"].T, p["conv_k"]).view(b, t, hq, hd)
    v = conv(xr @ p["v_proj.weight"].T, p["conv_v"]).view(b, t, hv, hd)
    a, bl = xr @ p["a_proj.weight"].T, xr @ p["b_proj.weight"].T
    g = -p["A_log"].exp() * F.softplus(a + p["dt_bias"])
    o, _ = recurrent_gated_delta_rule(F.normalize(q, dim=-1), F.normalize(k, dim=-1), v, g, bl.sigmoid(), hd**-0.5,
                                      cu_seqlens=cu)
    gate = (xr @ p["g_proj.weight"].T).view(b, t, hv, hd)
    o = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + layer.o_norm.eps) * p["o_norm.weight"] * F.silu(gate)
    out = o.flatten(-2) @ p["o_proj.weight"].T
    (out * cotangent.double()).sum().backward()
    return xr.grad, {n: v.grad for n, v in p.items()}


# the reference's options matrix for gradients (tests/model/test_gdn.py:104-162): GVA 1 and 2 x
# {documents of 1-3 tokens, one document over the window} x {in-kernel gate, torch gate}, plus rows
_CU_CASES = {"rows": None, "short_docs": [0, 1, 3, 4, 70, 200, 512], "one_doc": [0, 512]}


@pytest.mark.parametrize("kernel_gate", [True, False], ids=["kernel_gate", "torch_gate"])
@pytest.mark.parametrize("cu_case", sorted(_CU_CASES))
@pytest.mark.parametrize("rep", [1, 2], ids=["no_gva", "gva2x"])
def test_layer_backward_matches_oracle(rep, cu_case, kernel_gate):
    cu = _CU_CASES[cu_case]
    torch.manual_seed(0)
    cfg = GDNLayerConfig(d_model=128, gdn_qk_heads=2, gdn_v_heads=2 * rep, gdn_head_dim=64, gdn_kernel_gate=kernel_gate,
                         gdn_fla_conv=True, fused_norm_gate=True)
    layer = GatedDeltaNet(cfg)
    gen = torch.Generator().manual_seed(2)
    b = 2 if cu is None else 1
    x = torch.randn(b, 512, 128, generator=gen)
    cot = torch.randn(b, 512, 128, generator=gen)
    cu_t = None if cu is None else torch.tensor(cu)
    gx_ref, gp_ref = _oracle_layer_loss(layer, x, cot, cu_t)
    layer = layer.to(DEV)
    xd = x.to(DEV).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = layer(xd, cu_seqlens=None if cu_t is None else cu_t.to(DEV), cu_seqlens_cpu=cu_t)
    (out.float() * cot.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    errs = {"x": rel_l2(xd.grad, gx_ref)}
    for n, prm in layer.named_parameters():
        assert prm.grad is not None, f"{n}: no gradient"
        errs[n] = rel_l2(prm.grad, gp_ref[n])
    print("  rel L2:", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if v > 3e-2}
    assert not bad, f"gradients off: {bad}"


@pytest.mark.parametrize("cu", [None, [0, 1, 3, 4, 70, 200, 256]], ids=["rows", "short_docs"])
def test_layer_step_compiles_without_graph_breaks(cu):
    """``torch.compile(fullgraph=True)`` of a layer's forward + backward (a graph break raises); the
    compiled step's gradients match the eager step's."""
    torch.manual_seed(0)
    cfg = GDNLayerConfig(d_model=128, gdn_qk_heads=2, gdn_v_heads=4, gdn_head_dim=64, gdn_kernel_gate=True,
                         gdn_fla_conv=True, fused_norm_gate=True)
    layer = GatedDeltaNet(cfg).to(DEV)
    b = 2 if cu is None else 1
    x = torch.randn(b, 256, 128, generator=torch.Generator().manual_seed(3)).to(DEV)
    cu_t = None if cu is None else torch.tensor(cu)
    cu_d = None if cu_t is None else cu_t.to(DEV)

    def step(xx):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = layer(xx, cu_seqlens=cu_d, cu_seqlens_cpu=cu_t)
        return out.float().square().mean()

    grads = []
    for fn in (step, torch.compile(step, fullgraph=True, backend="aot_eager")):
        layer.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        fn(xx).backward()
        torch.cuda.synchronize()
        grads.append([xx.grad] + [p.grad for p in layer.parameters()])
    # the traced graph may place autocast's bf16 casts differently: equal to bf16 rounding, not bit-exact
    for a, b_ in zip(*grads):
        assert rel_l2(a, b_) <= 2e-2, rel_l2(a, b_)


def test_selective_checkpoint_policy_sees_the_gdn_ops():
    """The ops go through the dispatcher (``torch.ops.sorernn.*``), so a selective activation-checkpoint
    policy can save them. The reference notes that FLA's autograd functions bypass the dispatcher and
    are always recomputed (``sore/model/checkpointing.py:10-17``). With MUST_SAVE on the chunk op
    the checkpointed step equals the plain one."""
    import functools
    from torch.utils.checkpoint import CheckpointPolicy, checkpoint, create_selective_checkpoint_contexts

    torch.manual_seed(0)
    cfg = GDNLayerConfig(d_model=128, gdn_qk_heads=2, gdn_v_heads=4, gdn_head_dim=64, gdn_kernel_gate=True,
                         gdn_fla_conv=True, fused_norm_gate=True)
    layer = GatedDeltaNet(cfg).to(DEV)
    x = torch.randn(2, 192, 128, generator=torch.Generator().manual_seed(4)).to(DEV)
    seen = set()
    saved_ops = {torch.ops.sorernn.chunk_gated_delta_rule_fwd.default, torch.ops.sorernn.causal_conv1d_fwd.default}

    def policy(ctx, op, *args, **kwargs):
        if str(op).startswith("sorernn."):
            seen.add(str(op))
        return CheckpointPolicy.MUST_SAVE if op in saved_ops else CheckpointPolicy.PREFER_RECOMPUTE

    def fwd(xx):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return layer(xx).float().square().mean()

    grads = []
    for use_ckpt in (False, True):
        layer.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        if use_ckpt:
            loss = checkpoint(fwd, xx, use_reentrant=False,
                              context_fn=functools.partial(create_selective_checkpoint_contexts, policy))
        else:
            loss = fwd(xx)
        loss.backward()
        torch.cuda.synchronize()
        grads.append([xx.grad] + [p.grad for p in layer.parameters()])
    assert {"sorernn.chunk_gated_delta_rule_fwd.default", "sorernn.causal_conv1d_fwd.default",
            "sorernn.rms_norm_gated_fwd.default"} <= seen, seen
    for a, b_ in zip(*grads):
        assert rel_l2(a, b_) <= 2e-2, rel_l2(a, b_)
