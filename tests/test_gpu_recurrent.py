"""GPU parity: recurrent gated delta rule and the fused decode step vs the CPU oracle.

Every call goes through the C ABI of libgdn.so (``sorernn_amd.ops`` -> ctypes). Tolerances: the
BASELINE bar (max-abs 2e-2 on bf16 outputs, relative L2 1e-3 on fp32 final states).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import decode_step_ref, l2norm, recurrent_gated_delta_rule
from sorernn_amd import fused_recurrent_gated_delta_rule, gated_delta_decode_step
from sorernn_amd.synthetic import decode_inputs, gdn_inputs
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run_both(inp, **kw):
    d = inp.to(DEV)
    o, st = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                             output_final_state=True, cu_seqlens=d.cu_seqlens, **kw)
    torch.cuda.synchronize()
    return o.cpu(), st.cpu()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kd", [64, 128])
def test_recurrent_matches_oracle(dtype, kd):
    print(f"recurrent dtype={dtype} K=V={kd}", flush=True)
    inp = gdn_inputs(2, 37, 3, kd, dtype=dtype, seed=11, h0=True)
    o, st = _run_both(inp)
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    assert_output_close(o, o_ref)
    assert_state_close(st, st_ref)


def test_recurrent_single_token_closed_form():
    # T=1 from a zero state: o = scale (q.k) beta v
    inp = gdn_inputs(3, 1, 2, 128, dtype=torch.float32, seed=12)
    o, st = _run_both(inp)
    exp = inp.scale * (inp.q * inp.k).sum(-1, keepdim=True) * inp.beta[..., None] * inp.v
    assert_output_close(o, exp, tol=1e-5)
    exp_state = inp.k[:, 0, :, :, None] * (inp.beta[:, 0, :, None] * inp.v[:, 0])[:, :, None, :]
    assert_state_close(st, exp_state, tol=1e-5)


def test_recurrent_varlen_gva_and_kernel_options():
    cu = torch.tensor([0, 1, 2, 9, 40], dtype=torch.int32)
    inp = gdn_inputs(1, 40, 2, 64, HV=4, dtype=torch.bfloat16, seed=13, h0=True, cu_seqlens=cu)
    # raw gates: g holds a, beta holds logits; q/k unnormalised (normalised in the kernel)
    gen = torch.Generator().manual_seed(14)
    a = torch.randn(1, 40, 4, generator=gen)
    blog = torch.randn(1, 40, 4, generator=gen)
    A_log = torch.rand(4, generator=gen).mul(15).add(1).log()
    dt_bias = torch.randn(4, generator=gen) * 0.5
    q = (torch.randn(1, 40, 2, 64, generator=gen) * 3).to(torch.bfloat16)
    k = (torch.randn(1, 40, 2, 64, generator=gen) * 3).to(torch.bfloat16)
    d = lambda x: x.to(DEV)  # noqa: E731
    o, st = fused_recurrent_gated_delta_rule(
        d(q), d(k), d(inp.v), d(a), d(blog), scale=inp.scale, initial_state=d(inp.h0), output_final_state=True,
        cu_seqlens=d(cu), use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True, use_gate_in_kernel=True,
        A_log=d(A_log), dt_bias=d(dt_bias))
    g_ref = -A_log.exp() * F.softplus(a + dt_bias)
    qn = q.float() / q.float().norm(dim=-1, keepdim=True)
    kn = k.float() / k.float().norm(dim=-1, keepdim=True)
    o_ref, st_ref = recurrent_gated_delta_rule(qn, kn, inp.v.float(), g_ref, blog.sigmoid(), inp.scale, inp.h0, True,
                                               cu_seqlens=cu.long())
    assert_output_close(o.cpu(), o_ref.to(torch.bfloat16))
    assert_state_close(st.cpu(), st_ref)


def test_recurrent_inplace_state():
    inp = gdn_inputs(2, 5, 2, 128, dtype=torch.bfloat16, seed=15, h0=True)
    d = inp.to(DEV)
    h = d.h0.clone()
    o, st = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, initial_state=h, inplace_final_state=True)
    assert st.data_ptr() == h.data_ptr()
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(h.cpu(), st_ref)


@pytest.mark.parametrize("shape", [(4, 2, 2, 64), (64, 16, 16, 128), (3, 2, 4, 128)], ids=["small", "config2", "gva"])
def test_decode_step_matches_oracle(shape):
    b, h, hv, d = shape
    print(f"decode shape={shape}", flush=True)
    di = decode_inputs(B=b, H=h, HV=hv, D=d, seed=1002)
    dev = lambda x: x.to(DEV)  # noqa: E731
    conv, state = dev(di.conv_state), dev(di.state)
    o = gated_delta_decode_step(dev(di.x_qkv), conv, dev(di.conv_weight), dev(di.g), dev(di.beta), state, h, hv, d)
    torch.cuda.synchronize()
    o_ref, conv_ref, st_ref = decode_step_ref(di.x_qkv, di.conv_state, di.conv_weight, di.g, di.beta, di.state, h, hv, d)
    assert torch.equal(conv.cpu(), conv_ref), "conv cache must be shifted exactly"
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(state.cpu(), st_ref)


DECODE_OPTIONS = [
    # (activation dtype, gate/beta dtype, use_qk_l2norm, gate in kernel + beta sigmoid, D)
    (torch.float16, torch.float32, True, False, 128),
    (torch.float32, torch.float32, True, False, 128),
    (torch.bfloat16, torch.bfloat16, True, False, 128),
    (torch.bfloat16, torch.float32, False, False, 128),
    (torch.bfloat16, torch.float32, True, True, 128),
    (torch.bfloat16, torch.bfloat16, True, True, 64),
]


@pytest.mark.parametrize("dt,gdt,l2,kgate,d", DECODE_OPTIONS,
                         ids=["f16", "f32", "bf16_gates", "no_l2norm", "kernel_gate", "kernel_gate_bf16_d64"])
def test_decode_step_options_match_oracle(dt, gdt, l2, kgate, d):
    """The fused decode step over its input dtypes, 16-bit gates (the last element of g and beta is
    read at the tensors' final 2 bytes), the L2 norm on and off, and the in-kernel gate
    g = -exp(A_log) softplus(a + dt_bias) with beta = sigmoid(b) (oracle gate_and_beta), with GVA."""
    from oracle import gate_and_beta

    b, h, hv = 5, 2, 4
    print(f"decode options dt={dt} gates={gdt} l2={l2} kernel_gate={kgate} D={d}", flush=True)
    di = decode_inputs(B=b, H=h, HV=hv, D=d, dtype=dt, seed=1100 + d)
    gen = torch.Generator().manual_seed(7)
    if kgate:
        a_raw = torch.randn(b, hv, generator=gen).to(gdt)
        b_raw = torch.randn(b, hv, generator=gen).to(gdt)
        A_log = torch.rand(hv, generator=gen) * 2 - 1
        dt_bias = torch.randn(hv, generator=gen) * 0.5
        g_ref, beta_ref = gate_and_beta(a_raw[:, None], b_raw[:, None], A_log, dt_bias)
        g_ref, beta_ref = g_ref[:, 0], beta_ref[:, 0]
        g_in, beta_in = a_raw, b_raw
    else:
        g_in, beta_in = di.g.to(gdt), di.beta.to(gdt)
        g_ref, beta_ref = g_in.float(), beta_in.float()
    dev = lambda x: x.to(DEV)  # noqa: E731
    conv, state = dev(di.conv_state), dev(di.state)
    kw = dict(use_qk_l2norm_in_kernel=l2)
    if kgate:
        kw.update(use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, A_log=dev(A_log), dt_bias=dev(dt_bias))
    o = gated_delta_decode_step(dev(di.x_qkv), conv, dev(di.conv_weight), dev(g_in), dev(beta_in), state, h, hv, d, **kw)
    torch.cuda.synchronize()
    o_ref, conv_ref, st_ref = decode_step_ref(di.x_qkv, di.conv_state, di.conv_weight, g_ref, beta_ref, di.state,
                                              h, hv, d, use_qk_l2norm=l2)
    assert torch.equal(conv.cpu(), conv_ref), "conv cache must be shifted exactly"
    assert_output_close(o.cpu(), o_ref.to(dt))
    assert_state_close(state.cpu(), st_ref)


def test_decode_three_steps_in_a_row():
    di = decode_inputs(B=8, H=2, HV=2, D=128, seed=99)
    dev = lambda x: x.to(DEV)  # noqa: E731
    conv, state = dev(di.conv_state), dev(di.state)
    conv_r, st_r = di.conv_state.clone(), di.state.clone()
    gen = torch.Generator().manual_seed(5)
    for step in range(3):
        x = torch.randn(di.x_qkv.shape, generator=gen).to(di.x_qkv.dtype)
        o = gated_delta_decode_step(dev(x), conv, dev(di.conv_weight), dev(di.g), dev(di.beta), state, 2, 2, 128)
        o_r, conv_r, st_r = decode_step_ref(x, conv_r, di.conv_weight, di.g, di.beta, st_r, 2, 2, 128)
        assert_output_close(o.cpu(), o_r, what=f"o step {step}")
    assert torch.equal(conv.cpu(), conv_r)
    assert_state_close(state.cpu(), st_r)


def test_l2norm_in_recurrent_matches_prenormalised():
    # use_qk_l2norm_in_kernel on unnormalised inputs == pre-normalised inputs (fp32)
    gen = torch.Generator().manual_seed(21)
    q = torch.randn(1, 6, 2, 64, generator=gen) * 5
    k = torch.randn(1, 6, 2, 64, generator=gen) * 5
    inp = gdn_inputs(1, 6, 2, 64, dtype=torch.float32, seed=22, h0=True)
    d = lambda x: x.to(DEV)  # noqa: E731
    o1, s1 = fused_recurrent_gated_delta_rule(d(q), d(k), d(inp.v), d(inp.g), d(inp.beta), initial_state=d(inp.h0),
                                              output_final_state=True, use_qk_l2norm_in_kernel=True)
    o2, s2 = fused_recurrent_gated_delta_rule(d(l2norm(q)), d(l2norm(k)), d(inp.v), d(inp.g), d(inp.beta),
                                              initial_state=d(inp.h0), output_final_state=True)
    assert_output_close(o1.cpu(), o2.cpu(), tol=1e-5)
    assert_state_close(s1.cpu(), s2.cpu(), tol=1e-5)
