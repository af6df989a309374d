"""Pins for the CPU oracle (no GPU).

The reference's own known-answer tests for this path (``tests/model/test_gdn_ref.py``,
``test_conv.py``, ``test_varlen.py``, ``test_layers.py``) are restated here against the oracle,
together with checks the mathematics fixes: closed forms, an independent matrix-transition
formulation, split invariance, the chunked algebra in fp64 and brute force on tiny inputs.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import (
    causal_conv1d_silu,
    causal_conv1d_varlen,
    chunk_gated_delta_rule_bwd_ref,
    chunk_gated_delta_rule_ref,
    conv_state_from_sequence,
    decode_step_ref,
    doc_ids_from_cu_seqlens,
    gate_and_beta,
    l2norm,
    matrix_transition_rule,
    naive_gated_delta_rule,
    positions_from_cu_seqlens,
    recurrent_gated_delta_rule,
    rms_norm,
    rms_norm_gated,
)

DK, DV, H = 8, 6, 2


def _inputs(b, t, dtype=torch.float64, seed=0, h=H, dk=DK, dv=DV):
    """q,k L2-normalised; g <= 0; beta in (0,1) -- the reference's ``_inputs`` (test_gdn_ref.py:11-22)."""
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(b, t, h, dk, generator=gen, dtype=dtype), dim=-1)
    k = F.normalize(torch.randn(b, t, h, dk, generator=gen, dtype=dtype), dim=-1)
    v = torch.randn(b, t, h, dv, generator=gen, dtype=dtype)
    g = -torch.rand(b, t, h, generator=gen, dtype=dtype)
    beta = torch.rand(b, t, h, generator=gen, dtype=dtype)
    return q, k, v, g, beta


def _cu(values):
    return torch.tensor(values, dtype=torch.long)


# ---------------------------------------------------------------- reference KATs (test_gdn_ref.py)
def test_single_step_closed_form():
    # test_gdn_ref.py:29-37: T=1 from a zero state gives o = scale (q.k) beta v
    q, k, v, g, beta = _inputs(2, 1)
    out = naive_gated_delta_rule(q, k, v, g, beta, scale=0.37)
    expected = 0.37 * (q * k).sum(-1, keepdim=True) * beta[..., None] * v
    assert out.shape == (2, 1, H, DV)
    torch.testing.assert_close(out, expected, atol=1e-12, rtol=0)


def test_two_steps_hand_computed():
    # test_gdn_ref.py:40-53: decay before the update, read after the update
    q, k, v, g, beta = _inputs(1, 2, seed=1)
    out = naive_gated_delta_rule(q, k, v, g, beta, scale=0.5)
    h = torch.zeros(1, H, DK, DV, dtype=torch.float64)
    exp = []
    for t in range(2):
        h = h * g[:, t].exp()[..., None, None]
        d = (v[:, t] - torch.einsum("bhd,bhdm->bhm", k[:, t], h)) * beta[:, t, :, None]
        h = h + k[:, t, :, :, None] * d[:, :, None, :]
        exp.append(torch.einsum("bhd,bhdm->bhm", q[:, t] * 0.5, h))
    torch.testing.assert_close(out, torch.stack(exp, 1), atol=1e-12, rtol=0)


def test_varlen_equals_separate():
    q, k, v, g, beta = _inputs(1, 12, dtype=torch.float32, seed=2)
    s = DK**-0.5
    packed = naive_gated_delta_rule(q, k, v, g, beta, s, cu_seqlens=_cu([0, 5, 12]))
    first = naive_gated_delta_rule(q[:, :5], k[:, :5], v[:, :5], g[:, :5], beta[:, :5], s)
    second = naive_gated_delta_rule(q[:, 5:], k[:, 5:], v[:, 5:], g[:, 5:], beta[:, 5:], s)
    torch.testing.assert_close(packed, torch.cat([first, second], 1), atol=1e-6, rtol=0)


def test_varlen_resets_state_between_documents():
    q, k, v, g, beta = _inputs(1, 12, seed=3)
    s = DK**-0.5
    with_cu = naive_gated_delta_rule(q, k, v, g, beta, s, cu_seqlens=_cu([0, 5, 12]))
    without = naive_gated_delta_rule(q, k, v, g, beta, s)
    torch.testing.assert_close(with_cu[:, :5], without[:, :5], atol=1e-12, rtol=0)
    assert not torch.allclose(with_cu[:, 5:], without[:, 5:], atol=1e-3)


def test_varlen_single_token_documents():
    q, k, v, g, beta = _inputs(1, 4, seed=4)
    s = DK**-0.5
    packed = naive_gated_delta_rule(q, k, v, g, beta, s, cu_seqlens=_cu([0, 1, 2, 4]))
    parts = [naive_gated_delta_rule(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b], s) for a, b in [(0, 1), (1, 2), (2, 4)]]
    torch.testing.assert_close(packed, torch.cat(parts, 1), atol=1e-12, rtol=0)


def test_varlen_requires_batch_one():
    q, k, v, g, beta = _inputs(2, 6)
    with pytest.raises(ValueError, match="B == 1"):
        naive_gated_delta_rule(q, k, v, g, beta, 1.0, cu_seqlens=_cu([0, 3, 6]))


def test_varlen_rejects_cu_seqlens_not_covering_sequence():
    q, k, v, g, beta = _inputs(1, 6)
    with pytest.raises(ValueError, match="cu_seqlens"):
        naive_gated_delta_rule(q, k, v, g, beta, 1.0, cu_seqlens=_cu([0, 3, 5]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_input_returns_input_dtype(dtype):
    # test_gdn_ref.py:125-137: computed in fp32, returned in the input dtype
    q, k, v, g, beta = _inputs(1, 6, dtype=torch.float32, seed=6)
    lp = [x.to(dtype) for x in (q, k, v, g, beta)]
    out = naive_gated_delta_rule(*lp, scale=DK**-0.5)
    assert out.dtype == dtype
    ref = naive_gated_delta_rule(*[x.float() for x in lp], scale=DK**-0.5)
    torch.testing.assert_close(out.float(), ref.to(dtype).float(), atol=0, rtol=0)


# ---------------------------------------------------------------- extensions: h0 / final state
def test_one_step_from_state_closed_form():
    # T=1 from S0: o = scale (e^g S0^T q + delta (k.q)), delta = beta (v - e^g S0^T k)
    q, k, v, g, beta = _inputs(2, 1, seed=7)
    s0 = torch.randn(2, H, DK, DV, dtype=torch.float64, generator=torch.Generator().manual_seed(8))
    o, st = recurrent_gated_delta_rule(q, k, v, g, beta, 0.3, initial_state=s0, output_final_state=True)
    a = g[:, 0].exp()[..., None]  # [B,H,1]
    s0tk = torch.einsum("bhkv,bhk->bhv", s0, k[:, 0])
    s0tq = torch.einsum("bhkv,bhk->bhv", s0, q[:, 0])
    delta = beta[:, 0, :, None] * (v[:, 0] - a * s0tk)
    exp_o = 0.3 * (a * s0tq + delta * (k[:, 0] * q[:, 0]).sum(-1, keepdim=True))
    exp_s = a[..., None] * s0 + k[:, 0, :, :, None] * delta[:, :, None, :]
    torch.testing.assert_close(o[:, 0], exp_o, atol=1e-12, rtol=0)
    torch.testing.assert_close(st, exp_s, atol=1e-12, rtol=0)


def test_zero_initial_state_is_the_reference_recurrence():
    q, k, v, g, beta = _inputs(2, 9, seed=9)
    o1 = naive_gated_delta_rule(q, k, v, g, beta, 0.4)
    o2, _ = recurrent_gated_delta_rule(q, k, v, g, beta, 0.4, initial_state=torch.zeros(2, H, DK, DV, dtype=torch.float64))
    torch.testing.assert_close(o1, o2, atol=0, rtol=0)


@pytest.mark.parametrize("split", [1, 5, 12])
def test_split_invariance_pins_initial_and_final_state(split):
    q, k, v, g, beta = _inputs(2, 13, seed=10)
    s0 = 0.1 * torch.randn(2, H, DK, DV, dtype=torch.float64, generator=torch.Generator().manual_seed(11))
    o, st = recurrent_gated_delta_rule(q, k, v, g, beta, 0.35, s0, True)
    o1, s1 = recurrent_gated_delta_rule(q[:, :split], k[:, :split], v[:, :split], g[:, :split], beta[:, :split], 0.35, s0, True)
    sl = slice(split, None)
    o2, s2 = recurrent_gated_delta_rule(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], 0.35, s1, True)
    torch.testing.assert_close(torch.cat([o1, o2], 1), o, atol=1e-12, rtol=0)
    torch.testing.assert_close(s2, st, atol=1e-12, rtol=0)


def test_varlen_final_states_equal_separate_runs():
    q, k, v, g, beta = _inputs(1, 15, seed=12)
    bounds = [0, 1, 6, 15]
    s0 = torch.randn(3, H, DK, DV, dtype=torch.float64, generator=torch.Generator().manual_seed(13))
    o, st = recurrent_gated_delta_rule(q, k, v, g, beta, 0.3, s0, True, cu_seqlens=_cu(bounds))
    for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        on, sn = recurrent_gated_delta_rule(q[:, a:e], k[:, a:e], v[:, a:e], g[:, a:e], beta[:, a:e], 0.3, s0[n : n + 1], True)
        torch.testing.assert_close(o[:, a:e], on, atol=1e-12, rtol=0)
        torch.testing.assert_close(st[n : n + 1], sn, atol=1e-12, rtol=0)


def test_matrix_transition_form_matches_delta_form():
    q, k, v, g, beta = _inputs(2, 11, seed=14)
    s0 = torch.randn(2, H, DK, DV, dtype=torch.float64, generator=torch.Generator().manual_seed(15))
    o, st = recurrent_gated_delta_rule(q, k, v, g, beta, 0.3, s0, True)
    o2, st2 = matrix_transition_rule(q, k, v, g, beta, 0.3, s0)
    torch.testing.assert_close(o, o2, atol=1e-12, rtol=0)
    torch.testing.assert_close(st, st2, atol=1e-12, rtol=0)


def test_brute_force_tiny_scalar_loops():
    # K=2, V=1, T=3 written out with scalars only (no tensor algebra), from a known state
    q = [[0.6, 0.8], [1.0, 0.0], [0.0, -1.0]]
    k = [[0.8, 0.6], [0.0, 1.0], [0.6, -0.8]]
    v = [2.0, -1.0, 0.5]
    g = [-0.1, -0.5, 0.0]
    be = [0.5, 1.0, 0.25]
    s = [0.3, -0.2]  # state column (K=2, V=1)
    outs = []
    for t in range(3):
        a = math.exp(g[t])
        s = [a * s[0], a * s[1]]
        d = be[t] * (v[t] - (s[0] * k[t][0] + s[1] * k[t][1]))
        s = [s[0] + k[t][0] * d, s[1] + k[t][1] * d]
        outs.append(0.7 * (q[t][0] * s[0] + q[t][1] * s[1]))
    tq = torch.tensor(q, dtype=torch.float64).view(1, 3, 1, 2)
    tk = torch.tensor(k, dtype=torch.float64).view(1, 3, 1, 2)
    tv = torch.tensor(v, dtype=torch.float64).view(1, 3, 1, 1)
    tg = torch.tensor(g, dtype=torch.float64).view(1, 3, 1)
    tb = torch.tensor(be, dtype=torch.float64).view(1, 3, 1)
    s0 = torch.tensor([0.3, -0.2], dtype=torch.float64).view(1, 1, 2, 1)
    o, st = recurrent_gated_delta_rule(tq, tk, tv, tg, tb, 0.7, s0, True)
    torch.testing.assert_close(o.flatten(), torch.tensor(outs, dtype=torch.float64), atol=1e-14, rtol=0)
    torch.testing.assert_close(st.flatten(), torch.tensor(s, dtype=torch.float64), atol=1e-14, rtol=0)


def test_gva_equals_repeat_interleave():
    gen = torch.Generator().manual_seed(16)
    q = F.normalize(torch.randn(1, 7, 2, DK, generator=gen, dtype=torch.float64), dim=-1)
    k = F.normalize(torch.randn(1, 7, 2, DK, generator=gen, dtype=torch.float64), dim=-1)
    v = torch.randn(1, 7, 4, DV, generator=gen, dtype=torch.float64)
    g = -torch.rand(1, 7, 4, generator=gen, dtype=torch.float64)
    beta = torch.rand(1, 7, 4, generator=gen, dtype=torch.float64)
    o, _ = recurrent_gated_delta_rule(q, k, v, g, beta, 0.3)
    rep = lambda x: x.repeat_interleave(2, dim=2)  # noqa: E731
    o2, _ = recurrent_gated_delta_rule(rep(q), rep(k), v, g, beta, 0.3)
    torch.testing.assert_close(o, o2, atol=0, rtol=0)
    # head i of v reads q/k head i // 2: moving q head 1 changes v heads 2,3 only
    q2 = q.clone()
    q2[:, :, 1] = -q2[:, :, 1]
    o3, _ = recurrent_gated_delta_rule(q2, k, v, g, beta, 0.3)
    torch.testing.assert_close(o3[:, :, :2], o[:, :, :2], atol=0, rtol=0)
    assert not torch.allclose(o3[:, :, 2:], o[:, :, 2:])


# ---------------------------------------------------------------- chunked algebra
def _config0(seed=1000, t=256, h=4, d=64, h0=False, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(1, t, h, d, generator=gen), dim=-1)
    k = F.normalize(torch.randn(1, t, h, d, generator=gen), dim=-1)
    v = torch.randn(1, t, h, d, generator=gen)
    beta = torch.randn(1, t, h, generator=gen).sigmoid()
    g = -F.softplus(torch.randn(1, t, h, generator=gen)) * (torch.rand(1, t, h, generator=gen) * 3 - 4).exp()
    s0 = 0.02 * torch.randn(1, h, d, d, generator=gen) if h0 else None
    cast = lambda x: None if x is None else x.to(dtype)  # noqa: E731
    return [cast(x) for x in (q, k, v, g, beta, s0)]


@pytest.mark.parametrize("t", [256, 200, 64, 65, 1])
def test_chunked_equals_recurrent_fp64(t):
    q, k, v, g, beta, s0 = _config0(t=t, h0=True)
    o, st = recurrent_gated_delta_rule(q, k, v, g, beta, None, s0, True)
    oc, stc = chunk_gated_delta_rule_ref(q, k, v, g, beta, None, s0, True)
    torch.testing.assert_close(oc, o, atol=1e-10, rtol=0)
    torch.testing.assert_close(stc, st, atol=1e-10, rtol=0)


def test_chunked_varlen_equals_recurrent_fp64():
    q, k, v, g, beta, _ = _config0(t=300, seed=1001)
    cu = _cu([0, 1, 64, 130, 131, 300])
    s0 = 0.02 * torch.randn(5, 4, 64, 64, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    o, st = recurrent_gated_delta_rule(q, k, v, g, beta, None, s0, True, cu_seqlens=cu)
    oc, stc = chunk_gated_delta_rule_ref(q, k, v, g, beta, None, s0, True, cu_seqlens=cu)
    torch.testing.assert_close(oc, o, atol=1e-10, rtol=0)
    torch.testing.assert_close(stc, st, atol=1e-10, rtol=0)


def test_chunked_plausible_mistakes_are_caught():
    # A dropped decay inside the chunk or a transposed solve must move the result far beyond 1e-10.
    q, k, v, g, beta, s0 = _config0(t=128, h0=True)
    o, _ = recurrent_gated_delta_rule(q, k, v, g, beta, None, s0, True)
    o_nodecay, _ = chunk_gated_delta_rule_ref(q, k, v, torch.zeros_like(g), beta, None, s0, True)
    assert (o_nodecay - o).abs().max() > 1e-3
    o_wrongbeta, _ = chunk_gated_delta_rule_ref(q, k, v, g, beta.flip(1), None, s0, True)
    assert (o_wrongbeta - o).abs().max() > 1e-3


# ---------------------------------------------------------------- conv (test_conv.py)
def _conv1d_oracle(x, weight):
    c, kw = weight.shape
    t = x.shape[1]
    return F.conv1d(x.transpose(1, 2), weight[:, None, :], padding=kw - 1, groups=c)[..., :t].transpose(1, 2)


@pytest.mark.parametrize("kw", [1, 2, 4])
@pytest.mark.parametrize("t", [1, 3, 10])
def test_conv_matches_conv1d_single_doc(kw, t):
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(2, t, 5, generator=gen, dtype=torch.float64)
    w = torch.randn(5, kw, generator=gen, dtype=torch.float64)
    exp = _conv1d_oracle(x, w)
    torch.testing.assert_close(causal_conv1d_varlen(x, w, None), exp, atol=1e-12, rtol=0)
    torch.testing.assert_close(causal_conv1d_varlen(x, w, torch.zeros(t, dtype=torch.long)), exp, atol=1e-12, rtol=0)


def test_conv_tap_order():
    x = torch.zeros(1, 5, 1)
    x[0, 2, 0] = 1.0
    out = causal_conv1d_varlen(x, torch.tensor([[1.0, 10.0, 100.0]]), None)
    assert out[0, :, 0].tolist() == [0.0, 0.0, 100.0, 10.0, 1.0]


def test_conv_no_leak_and_varlen_equals_separate():
    gen = torch.Generator().manual_seed(2)
    cu = _cu([0, 2, 3, 9])
    ids = doc_ids_from_cu_seqlens(cu, 9)
    x = torch.randn(1, 9, 3, generator=gen, dtype=torch.float64)
    w = torch.randn(3, 4, generator=gen, dtype=torch.float64)
    packed = causal_conv1d_varlen(x, w, ids)
    parts = [causal_conv1d_varlen(x[:, a:b], w, None) for a, b in [(0, 2), (2, 3), (3, 9)]]
    torch.testing.assert_close(packed, torch.cat(parts, 1), atol=1e-12, rtol=0)


def test_conv_nonfinite_input_does_not_leak():
    ids = doc_ids_from_cu_seqlens(_cu([0, 4, 9]), 9)
    x = torch.randn(1, 9, 3, dtype=torch.float64)
    x[:, 3] = float("nan")
    out = causal_conv1d_varlen(x, torch.randn(3, 4, dtype=torch.float64), ids)
    assert torch.isfinite(out[:, 4:]).all() and torch.isnan(out[:, 3]).all()


def test_conv_silu_and_state():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 10, 4, generator=gen)
    w = torch.randn(4, 4, generator=gen)
    cu = _cu([0, 2, 10])
    y = causal_conv1d_silu(x, w, cu)
    ids = doc_ids_from_cu_seqlens(cu, 10)
    torch.testing.assert_close(y, F.silu(causal_conv1d_varlen(x.double(), w.double(), ids)).float(), atol=1e-6, rtol=0)
    st = conv_state_from_sequence(x, 4, cu)
    assert st.shape == (2, 4, 4)
    torch.testing.assert_close(st[0, :, 2:], x[0, 0:2].T)  # short doc: zero-padded at the front
    assert (st[0, :, :2] == 0).all()
    torch.testing.assert_close(st[1], x[0, 6:10].T)


# ---------------------------------------------------------------- varlen (test_varlen.py)
def test_doc_ids_positions():
    assert doc_ids_from_cu_seqlens(_cu([0, 3, 5]), 5).tolist() == [0, 0, 0, 1, 1]
    assert positions_from_cu_seqlens(_cu([0, 3, 5]), 5).tolist() == [0, 1, 2, 0, 1]
    cu = _cu([0, 1, 2, 5])
    assert doc_ids_from_cu_seqlens(cu, 5).tolist() == [0, 1, 2, 2, 2]
    assert positions_from_cu_seqlens(cu, 5).tolist() == [0, 0, 0, 1, 2]
    cu32 = torch.tensor([0, 3, 5], dtype=torch.int32)
    ids, pos = doc_ids_from_cu_seqlens(cu32, 5), positions_from_cu_seqlens(cu32, 5)
    assert ids.dtype == pos.dtype == torch.long
    assert ids.tolist() == [0, 0, 0, 1, 1] and pos.tolist() == [0, 1, 2, 0, 1]


# ---------------------------------------------------------------- norms and gates
def test_l2norm_matches_f_normalize():
    x = torch.randn(3, 5, 16, dtype=torch.float64)
    torch.testing.assert_close(l2norm(x), F.normalize(x, dim=-1), atol=1e-15, rtol=0)
    assert (l2norm(torch.zeros(2, 8)) == 0).all()


def test_rms_norm_formula():
    # test_layers.py:7-12
    x = torch.randn(2, 5, 16)
    ref = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    torch.testing.assert_close(rms_norm(x, torch.ones(16), 1e-6), ref)
    assert rms_norm(x.bfloat16(), torch.ones(16)).dtype == torch.bfloat16


def test_rms_norm_weight_known_values():
    """A row with a hand-computable RMS and a non-trivial weight: x = [3, 4, 0, 0] has mean(x^2) = 6.25,
    so with eps = 0 the normalised row is x / 2.5 = [1.2, 1.6, 0, 0], scaled elementwise by the weight;
    scaling x by any c > 0 leaves the output unchanged (eps = 0); a weight applied before the RMS (a
    planted mistake) would change mean(x^2) and is caught."""
    x = torch.tensor([[3.0, 4.0, 0.0, 0.0]], dtype=torch.float64)
    w = torch.tensor([2.0, -0.5, 7.0, 1.0], dtype=torch.float64)
    expected = torch.tensor([[2.4, -0.8, 0.0, 0.0]], dtype=torch.float64)
    torch.testing.assert_close(rms_norm(x, w, 0.0), expected, atol=1e-15, rtol=0)
    torch.testing.assert_close(rms_norm(37.5 * x, w, 0.0), expected, atol=1e-14, rtol=0)
    wrong = (x * w) * torch.rsqrt((x * w).pow(2).mean(-1, keepdim=True))
    assert (wrong - expected).abs().max() > 0.1
    # the gated form on the same row: silu(0) = 0; silu(40) = 40 sigmoid(40) = 40 to 1e-17 relative
    gate = torch.tensor([[0.0, 40.0, 1.0, 40.0]], dtype=torch.float64)
    got = rms_norm_gated(x, gate, w, 0.0)
    torch.testing.assert_close(got[0, 0], torch.tensor(0.0, dtype=torch.float64))
    torch.testing.assert_close(got[0, 1], torch.tensor(-0.8 * 40, dtype=torch.float64), atol=0, rtol=1e-14)


def test_rms_norm_gated_equals_norm_times_silu():
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(4, 3, 32, generator=gen, dtype=torch.float64)
    gate = torch.randn(4, 3, 32, generator=gen, dtype=torch.float64)
    w = torch.randn(32, generator=gen, dtype=torch.float64)
    exp = rms_norm(x, w, 1e-6) * gate * torch.sigmoid(gate)
    torch.testing.assert_close(rms_norm_gated(x, gate, w, 1e-6), exp, atol=1e-14, rtol=0)


def test_gate_and_beta_closed_form():
    A_log = torch.tensor([0.0, math.log(4.0)])
    dt_bias = torch.tensor([0.5, -1.0])
    a = -dt_bias.view(1, 1, 2).expand(1, 3, 2).clone()  # softplus(0) = log 2
    b = torch.zeros(1, 3, 2)
    g, beta = gate_and_beta(a, b, A_log, dt_bias)
    torch.testing.assert_close(g, -torch.tensor([1.0, 4.0]).view(1, 1, 2).expand(1, 3, 2) * math.log(2.0))
    torch.testing.assert_close(beta, torch.full((1, 3, 2), 0.5))
    a2 = torch.randn(2, 4, 2)
    g2, _ = gate_and_beta(a2, b[:, :1].expand(2, 4, 2), A_log, dt_bias)
    torch.testing.assert_close(g2, -A_log.exp() * F.softplus(a2 + dt_bias))


# ---------------------------------------------------------------- decode step
def test_decode_step_equals_last_token_of_sequence():
    gen = torch.Generator().manual_seed(21)
    b, h, d, t, width = 2, 2, 8, 6, 4
    c = 3 * h * d
    x = torch.randn(b, t, c, generator=gen)
    w = torch.randn(c, width, generator=gen) * 0.5
    a = -F.softplus(torch.randn(b, t, h, generator=gen))
    beta = torch.rand(b, t, h, generator=gen)
    s0 = 0.02 * torch.randn(b, h, d, d, generator=gen)
    # full-sequence reference: conv + SiLU (rounded once), fp32 L2 norm, recurrence
    y = F.silu(causal_conv1d_varlen(x.double(), w.double(), None)).float()
    q = y[..., : h * d].view(b, t, h, d)
    k = y[..., h * d : 2 * h * d].view(b, t, h, d)
    v = y[..., 2 * h * d :].view(b, t, h, d)
    o_full, s_full = recurrent_gated_delta_rule(F.normalize(q, dim=-1), F.normalize(k, dim=-1), v, a, beta, None, s0, True)
    # prefill t-1 tokens, then one decode step from the conv cache
    _, s_pre = recurrent_gated_delta_rule(
        F.normalize(q[:, :-1], dim=-1), F.normalize(k[:, :-1], dim=-1), v[:, :-1], a[:, :-1], beta[:, :-1], None, s0, True
    )
    cache = conv_state_from_sequence(x[:, :-1], width)
    o, new_cache, s = decode_step_ref(x[:, -1], cache, w, a[:, -1], beta[:, -1], s_pre, h, h, d)
    torch.testing.assert_close(o[:, 0], o_full[:, -1], atol=1e-5, rtol=0)
    torch.testing.assert_close(s, s_full, atol=1e-5, rtol=0)
    torch.testing.assert_close(new_cache, conv_state_from_sequence(x, width))


# ---------------------------------------------------------------- backward of the chunked rule
def _bwd_case(t, h, hv, kd, vd, seed, cu=None):
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(1, t, h, kd, generator=gen, dtype=torch.float64), dim=-1)
    k = F.normalize(torch.randn(1, t, h, kd, generator=gen, dtype=torch.float64), dim=-1)
    v = torch.randn(1, t, hv, vd, generator=gen, dtype=torch.float64)
    g = -torch.rand(1, t, hv, generator=gen, dtype=torch.float64) * 0.3
    beta = torch.rand(1, t, hv, generator=gen, dtype=torch.float64)
    n = 1 if cu is None else len(cu) - 1
    h0 = torch.randn(n, hv, kd, vd, generator=gen, dtype=torch.float64) * 0.1
    do = torch.randn(1, t, hv, vd, generator=gen, dtype=torch.float64)
    dht = torch.randn(n, hv, kd, vd, generator=gen, dtype=torch.float64)
    return q, k, v, g, beta, h0, do, dht


@pytest.mark.parametrize("case", [
    dict(t=150, h=2, hv=4, kd=8, vd=6, chunk=16, cu=[0, 40, 41, 150]),  # GVA, varlen, partial chunks
    dict(t=70, h=1, hv=1, kd=5, vd=3, chunk=64, cu=None),
    dict(t=33, h=2, hv=2, kd=4, vd=4, chunk=8, cu=[0, 1, 2, 33]),        # single-token documents
], ids=["gva_varlen", "plain", "short_docs"])
def test_chunk_bwd_equals_autograd_through_recurrence(case):
    """The chunk-form backward against torch autograd through the token recurrence (fp64)."""
    cu = None if case["cu"] is None else torch.tensor(case["cu"])
    q, k, v, g, beta, h0, do, dht = _bwd_case(case["t"], case["h"], case["hv"], case["kd"], case["vd"], 11, case["cu"])
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, g, beta, h0)]
    o, ht = recurrent_gated_delta_rule(*leaves[:5], scale=0.3, initial_state=leaves[5], output_final_state=True,
                                       cu_seqlens=cu)
    ref = torch.autograd.grad((o * do).sum() + (ht * dht).sum(), leaves)
    mine = chunk_gated_delta_rule_bwd_ref(q, k, v, g, beta, do, scale=0.3, initial_state=h0, dht=dht, cu_seqlens=cu,
                                          chunk_size=case["chunk"])
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), mine, ref):
        torch.testing.assert_close(a, b, rtol=0, atol=1e-10, msg=lambda m, n=name: f"{n}: {m}")


def test_chunk_bwd_plausible_mistakes_are_caught():
    """Each plausible slip in the backward (a dropped term, a sign) moves some gradient by O(1)."""
    q, k, v, g, beta, h0, do, dht = _bwd_case(40, 1, 1, 6, 5, 12)
    good = chunk_gated_delta_rule_bwd_ref(q, k, v, g, beta, do, 0.4, h0, dht, chunk_size=16)
    variants = {
        "no_dht": chunk_gated_delta_rule_bwd_ref(q, k, v, g, beta, do, 0.4, h0, None, chunk_size=16),
        "gate_sign": chunk_gated_delta_rule_bwd_ref(q, k, v, -g, beta, do, 0.4, h0, dht, chunk_size=16),
        "beta_off": chunk_gated_delta_rule_bwd_ref(q, k, v, g, beta * 0.5, do, 0.4, h0, dht, chunk_size=16),
    }
    for name, bad in variants.items():
        assert any(float((a - b).abs().max()) > 1e-3 for a, b in zip(good, bad)), name
    # the finite difference of the loss matches the analytic gradient in each input direction
    gen = torch.Generator().manual_seed(13)
    loss = lambda *xs: (recurrent_gated_delta_rule(*xs[:5], scale=0.4, initial_state=xs[5], output_final_state=True)[0] * do).sum() \
        + (recurrent_gated_delta_rule(*xs[:5], scale=0.4, initial_state=xs[5], output_final_state=True)[1] * dht).sum()  # noqa: E731
    base = [q, k, v, g, beta, h0]
    for i, grad in enumerate(good):
        d = torch.randn(base[i].shape, generator=gen, dtype=torch.float64)
        eps = 1e-6
        plus = [x + eps * d if j == i else x for j, x in enumerate(base)]
        minus = [x - eps * d if j == i else x for j, x in enumerate(base)]
        fd = (loss(*plus) - loss(*minus)) / (2 * eps)
        torch.testing.assert_close(fd, (grad * d).sum(), rtol=1e-6, atol=1e-8)
