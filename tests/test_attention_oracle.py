"""Pins for the attention oracle (no GPU): library routines, closed forms of the rotation, invariants.

The reference's own attention tests (``tests/model/test_attention.py``) need its module; here the
same properties are restated against ``oracle/attention_oracle.py``.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle.attention_oracle import causal_attention, gated_attention_layer, partial_rotary, rotary_cos_sin
from oracle.gdn_oracle import doc_ids_from_cu_seqlens, rms_norm


def _qkv(b=2, hq=4, hkv=2, t=37, d=16, dtype=torch.float64, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, hq, t, d, generator=g, dtype=dtype), torch.randn(b, hkv, t, d, generator=g, dtype=dtype),
            torch.randn(b, hkv, t, d, generator=g, dtype=dtype))


@pytest.mark.parametrize("hkv", [1, 2, 4])
def test_causal_attention_equals_sdpa(hkv):
    q, k, v = _qkv(hkv=hkv)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4 // hkv, 1), v.repeat_interleave(4 // hkv, 1),
                                         is_causal=True)
    torch.testing.assert_close(causal_attention(q, k, v), ref, atol=1e-12, rtol=0)


def test_document_mask_equals_sdpa_dense_mask_and_separate_runs():
    cu = torch.tensor([0, 5, 6, 30, 37])
    q, k, v = _qkv(b=1)
    ids = doc_ids_from_cu_seqlens(cu, 37)
    mask = torch.ones(37, 37, dtype=torch.bool).tril() & (ids[:, None] == ids[None, :])
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), attn_mask=mask)
    out = causal_attention(q, k, v, ids)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=0)
    for a, e in zip(cu[:-1].tolist(), cu[1:].tolist()):
        torch.testing.assert_close(out[:, :, a:e], causal_attention(q[:, :, a:e], k[:, :, a:e], v[:, :, a:e]),
                                   atol=1e-12, rtol=0)


def test_first_query_attends_only_to_itself():
    q, k, v = _qkv(hkv=4)
    torch.testing.assert_close(causal_attention(q, k, v)[:, :, 0], v[:, :, 0], atol=1e-12, rtol=0)


def test_rotary_position_zero_is_identity_and_tail_passes():
    x = torch.randn(1, 3, 2, 32, dtype=torch.float64)
    out = partial_rotary(x, torch.tensor([0, 5, 9]), rot_dim=8, theta=1e6)
    torch.testing.assert_close(out[:, 0], x[:, 0], atol=0, rtol=0)
    torch.testing.assert_close(out[..., 8:], x[..., 8:], atol=0, rtol=0)


def test_rotary_pairs_keep_norm_and_angle_is_position_times_frequency():
    rot, theta = 8, 1e6
    x = torch.randn(1, 1, 1, rot, dtype=torch.float64)
    pos = 7
    out = partial_rotary(x, torch.tensor([pos]), rot, theta)[0, 0, 0]
    xs = x[0, 0, 0]
    half = rot // 2
    for f in range(half):
        # (x_f, x_{f+half}) is rotated by angle pos * theta^(-2f/rot) (fp32 frequency math)
        ang = float(torch.tensor(pos, dtype=torch.float32) * (1.0 / theta ** torch.tensor(2 * f / rot, dtype=torch.float32)))
        a, c = float(xs[f]), float(xs[f + half])
        exp0 = a * math.cos(ang) - c * math.sin(ang)
        exp1 = c * math.cos(ang) + a * math.sin(ang)
        assert abs(float(out[f]) - exp0) < 1e-6 and abs(float(out[f + half]) - exp1) < 1e-6
        assert abs(math.hypot(float(out[f]), float(out[f + half])) - math.hypot(a, c)) < 1e-6


def test_rotary_scores_depend_only_on_position_difference():
    q = torch.randn(1, 1, 1, 16, dtype=torch.float64)
    k = torch.randn(1, 1, 1, 16, dtype=torch.float64)
    dot = lambda m, n: float((partial_rotary(q, torch.tensor([m]), 16, 1e4) * partial_rotary(k, torch.tensor([n]), 16, 1e4)).sum())  # noqa: E731
    # equal up to the fp32 rounding of the angles (position * frequency)
    assert abs(dot(10, 3) - dot(107, 100)) < 1e-4
    assert abs(dot(10, 3) - dot(10, 4)) > 1e-2


def test_planted_rotation_sign_error_is_caught():
    x = torch.randn(1, 1, 1, 8, dtype=torch.float64)
    cos, sin = rotary_cos_sin(torch.tensor([3]), 8, 1e6, torch.float64)
    rotated_wrong = torch.cat((x[..., 4:], -x[..., :4]), dim=-1)  # sign flipped
    wrong = x * cos[None, :, None] + rotated_wrong * sin[None, :, None]
    assert (wrong - partial_rotary(x, torch.tensor([3]), 8, 1e6)).abs().max() > 1e-3


def test_rotary_rejects_bad_rot_dim():
    with pytest.raises(ValueError):
        partial_rotary(torch.zeros(1, 1, 1, 8), torch.tensor([0]), 3, 1e6)


def test_layer_composition_matches_the_pinned_parts():
    g = torch.Generator().manual_seed(3)
    d, hq, hkv, dh, t = 32, 4, 2, 8, 11
    names = {"q_proj.weight": (hq * dh, d), "gate_proj.weight": (hq * dh, d), "k_proj.weight": (hkv * dh, d),
             "v_proj.weight": (hkv * dh, d), "o_proj.weight": (d, hq * dh), "q_norm.weight": (dh,), "k_norm.weight": (dh,)}
    w = {n: 0.2 * torch.randn(*s, generator=g, dtype=torch.float64) for n, s in names.items()}
    x = torch.randn(1, t, d, generator=g, dtype=torch.float64)
    cu = torch.tensor([0, 4, 11])
    out = gated_attention_layer(x, w, hq, hkv, dh, rot_dim=4, theta=1e6, cu_seqlens=cu)
    # the same layer, document by document, with positions restarting at 0
    parts = []
    for a, e in ((0, 4), (4, 11)):
        xs = x[:, a:e]
        q = rms_norm((xs @ w["q_proj.weight"].T).view(1, e - a, hq, dh), w["q_norm.weight"])
        k = rms_norm((xs @ w["k_proj.weight"].T).view(1, e - a, hkv, dh), w["k_norm.weight"])
        v = (xs @ w["v_proj.weight"].T).view(1, e - a, hkv, dh)
        pos = torch.arange(e - a)
        q, k = partial_rotary(q, pos, 4, 1e6), partial_rotary(k, pos, 4, 1e6)
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2).repeat_interleave(2, 1),
                                           v.transpose(1, 2).repeat_interleave(2, 1), is_causal=True)
        o = o.transpose(1, 2).reshape(1, e - a, hq * dh)
        parts.append((o * torch.sigmoid(xs @ w["gate_proj.weight"].T)) @ w["o_proj.weight"].T)
    torch.testing.assert_close(out, torch.cat(parts, 1), atol=1e-12, rtol=0)
