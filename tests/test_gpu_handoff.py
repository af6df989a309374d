"""GPU: the prefill -> decode handoff.

A prefill of the first T-1 tokens (``causal_conv1d(..., output_final_state=True)`` for the conv
cache, ``chunk_gated_delta_rule(..., output_final_state=True)`` for the state) followed by one fused
``gated_delta_decode_step`` on token T must reproduce the full-sequence prefill's last token: its
output within BASELINE's bf16 bar, its final state within the fp32 bar, and the conv cache exactly
(the cache holds raw inputs, newest last). The decode step's definition is the T = 1 case of the
recurrence (sore/model/gdn_ref.py:17-21) with the conv tap orientation of sore/model/conv.py:7; the
same chain is pinned on the CPU by tests/test_oracle.py::test_decode_step_equals_last_token_of_sequence.
The full-sequence output is also checked against the oracle.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import causal_conv1d_silu, l2norm, recurrent_gated_delta_rule
from sorernn_amd import causal_conv1d, chunk_gated_delta_rule, gated_delta_decode_step
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("rep", [1, 2], ids=["no_gva", "gva2x"])
@pytest.mark.parametrize("t", [65, 300], ids=lambda t: f"T{t}")
def test_prefill_then_decode_equals_full_sequence(t, rep):
    gen = torch.Generator().manual_seed(40 + t + rep)
    b, h, d, w = 3, 2, 128, 4
    hv = h * rep
    c = (2 * h + hv) * d
    x = torch.randn(b, t, c, generator=gen).to(torch.bfloat16)
    cw = (torch.rand(c, w, generator=gen) * 2 - 1) * w**-0.5
    g = -F.softplus(torch.randn(b, t, hv, generator=gen)) * (torch.rand(b, t, hv, generator=gen) * 3 - 4).exp()
    beta = torch.randn(b, t, hv, generator=gen).sigmoid()
    s0 = 0.02 * torch.randn(b, hv, d, d, generator=gen)
    xd, cwd, gd, bd, s0d = x.to(DEV), cw.to(DEV), g.to(DEV), beta.to(DEV), s0.to(DEV)

    def split(y, n):
        return (y[..., : h * d].reshape(b, n, h, d), y[..., h * d: 2 * h * d].reshape(b, n, h, d),
                y[..., 2 * h * d:].reshape(b, n, hv, d))

    # full sequence
    y, cache_full = causal_conv1d(xd, cwd, activation="silu", output_final_state=True)
    q, k, v = split(y, t)
    o_full, s_full = chunk_gated_delta_rule(q, k, v, gd, bd, initial_state=s0d, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    # prefill T-1 tokens, then one decode step
    y_pre, cache = causal_conv1d(xd[:, :-1], cwd, activation="silu", output_final_state=True)
    qp, kp, vp = split(y_pre, t - 1)
    _, state = chunk_gated_delta_rule(qp, kp, vp, gd[:, :-1], bd[:, :-1], initial_state=s0d, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)
    o_dec = gated_delta_decode_step(xd[:, -1], cache, cwd, gd[:, -1], bd[:, -1], state, h, hv, d)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu(), cache_full.cpu()), "conv cache after the decode step"
    assert_output_close(o_dec.cpu()[:, 0], o_full.cpu()[:, -1].float(), what="decoded token vs prefill")
    assert_state_close(state.cpu(), s_full.cpu(), what="state after the decode step")
    # the full-sequence prefill against the oracle (conv + SiLU rounded to bf16, fp32 L2 norm)
    yr = causal_conv1d_silu(x, cw)
    qr, kr, vr = (z.cpu() for z in split(yr, t))
    o_ref, s_ref = recurrent_gated_delta_rule(l2norm(qr), l2norm(kr), vr, g, beta, d**-0.5, s0, True)
    assert_output_close(o_dec.cpu()[:, 0], o_ref[:, -1].float(), what="decoded token vs oracle")
    assert_state_close(state.cpu(), s_ref, what="decode state vs oracle")
