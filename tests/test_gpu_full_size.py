"""GPU parity at BASELINE's full sizes, checked against the CPU oracle on slices the oracle finishes
in seconds.

- Config 3 (8 packed documents, 32768 tokens): the whole op runs once; its outputs and final states
  for the 1,112-token and the 9,480-token documents (two value heads each) are compared with the
  oracle's recurrence over those documents from their own initial states.
- Config 4's chunked op alone (B=2, T=8192, H=16, d=128, config 1's input distributions, initial
  states): every output and final state against the oracle's recurrence, at BASELINE's absolute
  bars (128-chunk chains, twice config 1's).
- Config 4's GDN layer (B=2, T=8192, hidden 2048, 16 heads of 128, in-kernel gate): the full layer
  runs on both routes (the fused inference route and the reference-expression route); the input of
  its o_proj (the gated RMSNorm of the delta rule's output) is captured and compared, for batch row
  1 and value heads 0 and 15, with the oracle composition of those heads (their projections, conv +
  SiLU, L2 norm, gate, recurrence over all 8192 tokens, gated RMSNorm).
- Config 4's gated attention layer (B=2, T=8192, 16 q / 4 kv heads, d=128): the input of its o_proj
  (gated attention output) on selected query rows against the oracle composition of those rows
  (projections, q/k RMSNorm, partial RoPE, causal softmax over the row's prefix, sigmoid gate).
Tolerances: BASELINE's max-abs 2e-2 on bf16 outputs, relative L2 1e-3 on fp32 final states.
"""
import pytest
import torch

from oracle import causal_conv1d_silu, gate_and_beta, l2norm, recurrent_gated_delta_rule, rms_norm_gated
from oracle.attention_oracle import partial_rotary
from oracle.gdn_oracle import rms_norm
from sorernn_amd import chunk_gated_delta_rule
from sorernn_amd.synthetic import config_inputs
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16


def test_config3_documents_match_oracle():
    inp = config_inputs(3)
    cu = inp.cu_seqlens
    lens = (cu[1:] - cu[:-1]).tolist()
    print("config3 lengths", lens, flush=True)
    d = inp.to(DEV)
    o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                   output_final_state=True, cu_seqlens=d.cu_seqlens, cu_seqlens_cpu=cu)
    torch.cuda.synchronize()
    o, st = o.cpu(), st.cpu()
    heads = [3, 12]
    for length in (1112, 9480):
        n = lens.index(length)
        a, e = int(cu[n]), int(cu[n + 1])
        sl = lambda x: x[:, a:e, heads]  # noqa: E731
        o_ref, st_ref = recurrent_gated_delta_rule(sl(inp.q), sl(inp.k), sl(inp.v), sl(inp.g), sl(inp.beta),
                                                   inp.scale, inp.h0[n:n + 1, heads], True)
        assert_output_close(o[:, a:e, heads], o_ref, what=f"o of document {n} ({length} tokens)")
        assert_state_close(st[n:n + 1, heads], st_ref, what=f"final state of document {n}")


def test_config4_chunk_op_matches_oracle():
    from sorernn_amd.synthetic import gdn_inputs

    inp = gdn_inputs(2, 8192, 16, 128, dtype=BF16, seed=1004, h0=True)
    print("config-4 chunk op: B=2, T=8192, H=16, d=128", flush=True)
    d = inp.to(DEV)
    o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                   output_final_state=True)
    torch.cuda.synchronize()
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    err = assert_output_close(o.cpu(), o_ref)
    rel = assert_state_close(st.cpu(), st_ref)
    print(f"  max-abs {err:.3e} (max|ref| {o_ref.abs().max().item():.2f}), state relative L2 {rel:.2e}", flush=True)


def _gdn_layer_config4():
    from sorernn_amd.gdn_layer import GatedDeltaNet, GDNLayerConfig

    torch.manual_seed(4)
    cfg = GDNLayerConfig(d_model=2048, gdn_qk_heads=16, gdn_v_heads=16, gdn_head_dim=128, gdn_kernel_gate=True,
                         gdn_fla_conv=True, fused_norm_gate=True)
    layer = GatedDeltaNet(cfg)
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "g_proj", "a_proj", "b_proj", "o_proj"):
            getattr(layer, name).weight.normal_(0, 0.02)
    return layer


def _capture_o_proj_input(layer):
    seen = {}

    def hook(_mod, args):
        seen["x"] = args[0].detach()

    return layer.o_proj.register_forward_pre_hook(hook), seen


def _gdn_heads_oracle(layer, x, row, heads):
    """The oracle composition of the GDN layer for value heads `heads` of batch row `row` (q/k head =
    value head here: 16 of each): bf16 projections, conv + SiLU rounded to bf16, fp32 L2 norm, gate,
    recurrence and gated RMSNorm, the rounding points of the GPU route."""
    hd = layer.head_dim
    xb = x[row:row + 1].to(BF16).float()
    cols = lambda h: slice(h * hd, (h + 1) * hd)  # noqa: E731

    def lin(w, rows):  # bf16 GEMM, bf16 output
        return (xb @ w[rows].to(BF16).float().T).to(BF16)

    outs = []
    with torch.no_grad():
        for h in heads:
            c = cols(h)
            q = causal_conv1d_silu(lin(layer.q_proj.weight, c), layer.conv_q[c].float())
            k = causal_conv1d_silu(lin(layer.k_proj.weight, c), layer.conv_k[c].float())
            v = causal_conv1d_silu(lin(layer.v_proj.weight, c), layer.conv_v[c].float())
            a = lin(layer.a_proj.weight, slice(h, h + 1))
            b = lin(layer.b_proj.weight, slice(h, h + 1))
            g, beta = gate_and_beta(a, b, layer.A_log[h:h + 1], layer.dt_bias[h:h + 1])
            t = x.shape[1]
            o, _ = recurrent_gated_delta_rule(l2norm(q.view(1, t, 1, hd)), l2norm(k.view(1, t, 1, hd)),
                                              v.view(1, t, 1, hd), g, beta, hd**-0.5)
            gate = lin(layer.g_proj.weight, c).view(1, t, 1, hd)
            outs.append(rms_norm_gated(o, gate, layer.o_norm.weight, layer.o_norm.eps))
    return torch.cat(outs, dim=2)  # [1, T, len(heads), hd]


@pytest.mark.parametrize("route", ["fused", "reference"])
def test_config4_gdn_layer_full_size_matches_oracle_heads(route):
    layer = _gdn_layer_config4()
    x = torch.randn(2, 8192, 2048, generator=torch.Generator().manual_seed(44))
    row, heads = 1, [0, 15]
    ref = _gdn_heads_oracle(layer, x, row, heads)
    layer = layer.to(DEV)
    handle, seen = _capture_o_proj_input(layer)
    try:
        with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
            xd = x.to(DEV)
            out = layer(xd) if route == "fused" else layer._forward_reference(xd)
        torch.cuda.synchronize()
    finally:
        handle.remove()
    assert torch.isfinite(out).all()
    got = seen["x"].view(2, 8192, 16, 128)[row:row + 1, :, heads].float().cpu()
    # the gated RMSNorm output is O(1-10) per element (unit RMS times silu(gate)): the layer bar of
    # tests/test_gpu_layer.py, max-abs <= 2e-2 max|ref|, and a relative L2 bound
    err, scale = (got - ref.float()).abs().max().item(), ref.float().abs().max().item()
    rel = ((got.double() - ref.double()).norm() / ref.double().norm()).item()
    print(f"  {route}: max-abs {err:.3e} (max|ref| {scale:.2f}), relative L2 {rel:.2e}", flush=True)
    assert torch.isfinite(got).all()
    assert err <= 2e-2 * scale, f"{route} route: max-abs {err:.3e} > 2e-2 * {scale:.3e}"
    assert rel <= 1e-2, f"{route} route: relative L2 {rel:.3e}"


def test_config4_attention_layer_full_size_rows():
    from sorernn_amd.attention import AttnLayerConfig, GatedAttention

    torch.manual_seed(5)
    cfg = AttnLayerConfig(d_model=2048, attn_heads=16, attn_kv_heads=4, attn_head_dim=128, rope_theta=1e6,
                          rope_partial=0.25)
    layer = GatedAttention(cfg)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1 + 0.1 * torch.randn_like(p))
            else:
                p.normal_(0, 0.02)
    b, t, hq, hkv, dh = 2, 8192, 16, 4, 128
    x = torch.randn(b, t, 2048, generator=torch.Generator().manual_seed(45))
    layer = layer.to(DEV)
    handle, seen = _capture_o_proj_input(layer)
    try:
        with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
            layer(x.to(DEV))
        torch.cuda.synchronize()
    finally:
        handle.remove()
    got = seen["x"].float().cpu()  # [B, T, HQ * D]
    w = {n: p.detach().cpu() for n, p in layer.state_dict().items()}
    rows, bi = [0, 1, 127, 128, 4095, 8191], 1
    xb = x[bi].to(BF16)
    lin = lambda name, a: a @ w[name].to(BF16).T  # noqa: E731  bf16 in, bf16 out
    last = max(rows) + 1
    with torch.no_grad():
        k = rms_norm(lin("k_proj.weight", xb[:last]).view(1, last, hkv, dh), w["k_norm.weight"])
        k = partial_rotary(k, torch.arange(last), layer.rotary.rot_dim, 1e6)[0]           # [T, HKV, D]
        v = lin("v_proj.weight", xb[:last]).view(last, hkv, dh)
        rep = hq // hkv
        for r in rows:
            q = rms_norm(lin("q_proj.weight", xb[r:r + 1]).view(1, 1, hq, dh), w["q_norm.weight"])
            q = partial_rotary(q, torch.tensor([r]), layer.rotary.rot_dim, 1e6)[0, 0].float()  # [HQ, D]
            kr = k[: r + 1].float().repeat_interleave(rep, 1)
            vr = v[: r + 1].float().repeat_interleave(rep, 1)
            s = torch.einsum("hd,thd->ht", q, kr) * dh**-0.5
            o = torch.einsum("ht,thd->hd", torch.softmax(s, -1), vr).to(BF16).reshape(hq * dh)
            ref = o.float() * torch.sigmoid(lin("gate_proj.weight", xb[r:r + 1]).float()[0])
            assert_output_close(got[bi, r].to(BF16), ref, what=f"attention output row {r}")
    print("attention rows checked", rows, flush=True)

