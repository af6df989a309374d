"""GPU parity of the gated attention layer's kernels (``gdn_attn_qk_norm_rope_fwd``, ``gdn_attn_fwd``)
and of the ``GatedAttention`` layer, against the CPU attention oracle on identical bf16 inputs.

Bars: the attention output is bf16, held to BASELINE's max-abs 2e-2 against the fp32 oracle; the
prologue follows the reference's rounding points, so nearly every element is bit-identical (the
rest differ by the last bit of a bf16 cos/sin or product).
"""
import pytest
import torch

from oracle.attention_oracle import causal_attention, gated_attention_layer, partial_rotary
from oracle.gdn_oracle import doc_ids_from_cu_seqlens, positions_from_cu_seqlens, rms_norm
from tests.parity import assert_output_close

DEV = "cuda:0"


def _randn(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(*shape, generator=g)).to(torch.bfloat16)


def _ref_rope(x, w, rot, theta, positions):
    # the reference's bf16 pipeline: RMSNorm rounded to bf16, then the rotary in bf16 arithmetic
    return partial_rotary(rms_norm(x, w), positions, rot, theta)


@pytest.mark.gpu
@pytest.mark.parametrize("rot,theta,wdt", [(32, 1e6, torch.float32), (128, 1e6, torch.bfloat16), (16, 1e7, torch.float32)])
@pytest.mark.parametrize("varlen", [False, True])
def test_qk_norm_rope_matches_oracle(rot, theta, wdt, varlen):
    from sorernn_amd.attention import attn_qk_norm_rope

    d, hq, hkv = 128, 4, 2
    b, t = (1, 333) if varlen else (2, 300)
    # q and k as column slices of one wider projection output (row stride > width)
    proj = _randn(b, t, (2 * hq + 2 * hkv) * d, seed=1, scale=3.0)
    q_in, k_in = proj[..., : hq * d], proj[..., 2 * hq * d: (2 * hq + hkv) * d]
    qw = (1 + 0.1 * torch.randn(d, generator=torch.Generator().manual_seed(2))).to(wdt)
    kw = (1 + 0.1 * torch.randn(d, generator=torch.Generator().manual_seed(3))).to(wdt)
    cu = torch.tensor([0, 5, 70, 200, 333]) if varlen else None
    pos = positions_from_cu_seqlens(cu, t) if varlen else torch.arange(t)
    q, k = attn_qk_norm_rope(q_in.to(DEV), k_in.to(DEV), qw.to(DEV), kw.to(DEV), hq, hkv, rot, theta, 1e-6,
                             None if cu is None else cu.to(DEV), cu)
    q_ref = _ref_rope(q_in.view(b, t, hq, d), qw, rot, theta, pos)
    k_ref = _ref_rope(k_in.view(b, t, hkv, d), kw, rot, theta, pos)
    for out, ref, nm in ((q, q_ref, "q"), (k, k_ref, "k")):
        out = out.cpu()
        assert out.shape == ref.shape
        assert_output_close(out, ref, what=nm)
        frac = (out != ref).float().mean().item()
        assert frac <= 5e-3, f"{nm}: {frac:.2%} of elements differ from the reference rounding"


def _attn_ref(q, k, v, gate, cu=None):
    """fp32 oracle of gdn_attn_fwd on the same bf16 inputs: [B,T,HQ*D] fp32."""
    b, t, hq, d = q.shape
    hkv = k.shape[2]
    ids = doc_ids_from_cu_seqlens(cu, t) if cu is not None else None
    o = causal_attention(q.float().transpose(1, 2), k.float().transpose(1, 2),
                         v.float().view(b, t, hkv, d).transpose(1, 2), ids)
    return o.transpose(1, 2).reshape(b, t, hq * d) * torch.sigmoid(gate.float())


def _attn_inputs(b, t, hq, hkv, d, seed, qscale=1.0):
    q = _randn(b, t, hq, d, seed=seed, scale=qscale)
    k = _randn(b, t, hkv, d, seed=seed + 1)
    wide = _randn(b, t, hkv * d + hq * d + 64, seed=seed + 2)  # v | gate | pad: strided views
    v, gate = wide[..., : hkv * d], wide[..., hkv * d: hkv * d + hq * d]
    return q, k, v, gate


@pytest.mark.gpu
@pytest.mark.parametrize("b,t,hq,hkv,d", [(2, 1, 4, 2, 128), (2, 63, 4, 1, 128), (1, 128, 2, 2, 128),
                                          (2, 129, 4, 2, 64), (1, 300, 8, 2, 128), (2, 517, 4, 4, 64)])
def test_attention_matches_oracle(b, t, hq, hkv, d):
    from sorernn_amd.attention import gated_attention

    q, k, v, gate = _attn_inputs(b, t, hq, hkv, d, seed=10 + t)
    o = gated_attention(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV))
    assert o.dtype == torch.bfloat16 and o.shape == (b, t, hq * d)
    assert_output_close(o.cpu(), _attn_ref(q, k, v, gate))


@pytest.mark.gpu
def test_attention_sharp_scores():
    """Large logits (q x 8): the running max changes across key blocks and must rescale exactly."""
    from sorernn_amd.attention import gated_attention

    q, k, v, gate = _attn_inputs(1, 400, 4, 2, 128, seed=7, qscale=8.0)
    o = gated_attention(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV))
    assert_output_close(o.cpu(), _attn_ref(q, k, v, gate))


@pytest.mark.gpu
def test_attention_late_dominant_keys():
    """Keys whose scores exceed every earlier key's by far more than the lazy-rescale margin arrive
    in a late block (keys 300-309 scaled x40): the rows that see them must move their reference max
    and rescale the sums accumulated over the earlier blocks; rows before them must not change."""
    from sorernn_amd.attention import gated_attention

    q, k, v, gate = _attn_inputs(1, 400, 4, 2, 128, seed=8)
    k = k.clone()
    k[:, 300:310] = (k[:, 300:310].float() * 40.0).to(torch.bfloat16)
    o = gated_attention(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV))
    assert_output_close(o.cpu(), _attn_ref(q, k, v, gate))


@pytest.mark.gpu
def test_attention_rejects_non_positive_scale():
    from sorernn_amd.attention import gated_attention

    q, k, v, gate = _attn_inputs(1, 64, 2, 1, 64, seed=9)
    for bad in (0.0, -0.125, float("inf")):
        with pytest.raises(ValueError, match="scale"):
            gated_attention(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV), scale=bad)


@pytest.mark.gpu
@pytest.mark.parametrize("cu_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("bounds", [[0, 5, 70, 200, 333], [0, 1, 2, 3, 129, 130, 333], [0, 333]])
def test_attention_varlen_matches_oracle(bounds, cu_dtype):
    from sorernn_amd.attention import gated_attention

    t = bounds[-1]
    cu = torch.tensor(bounds, dtype=cu_dtype)
    q, k, v, gate = _attn_inputs(1, t, 4, 2, 128, seed=20)
    o = gated_attention(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV), cu.to(DEV), cu)
    assert_output_close(o.cpu(), _attn_ref(q, k, v, gate, cu.long()))


@pytest.mark.gpu
def test_attention_full_block_pair_size_rows():
    """Config-4 size (B=2, T=8192, 16 q / 4 kv heads, d=128): selected query rows against a per-row
    oracle (each row needs only its own prefix of keys), including the first and last rows of the
    sequence and rows on both sides of a 128-query tile edge."""
    from sorernn_amd.attention import gated_attention

    b, t, hq, hkv, d = 2, 8192, 16, 4, 128
    q, k, v, gate = _attn_inputs(b, t, hq, hkv, d, seed=30)
    o = gated_attention(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV)).cpu()
    assert torch.isfinite(o.float()).all()
    rows = [0, 1, 127, 128, 4095, 5000, 8190, 8191]
    rep = hq // hkv
    for bi in range(b):
        for r in rows:
            qr = q[bi, r].float()                                     # [HQ, D]
            kr = k[bi, : r + 1].float().repeat_interleave(rep, 1)     # [r+1, HQ, D]
            vr = v[bi, : r + 1].float().view(r + 1, hkv, d).repeat_interleave(rep, 1)
            s = torch.einsum("hd,thd->ht", qr, kr) * d**-0.5
            ref = torch.einsum("ht,thd->hd", torch.softmax(s, -1), vr).reshape(hq * d) * torch.sigmoid(gate[bi, r].float())
            assert_output_close(o[bi, r], ref, what=f"o[{bi},{r}]")


def _layer(d_model, hq, hkv, dh, partial, theta, seed):
    from sorernn_amd.attention import AttnLayerConfig, GatedAttention

    torch.manual_seed(seed)
    layer = GatedAttention(AttnLayerConfig(d_model=d_model, attn_heads=hq, attn_kv_heads=hkv, attn_head_dim=dh,
                                           rope_theta=theta, rope_partial=partial))
    with torch.no_grad():
        for n, p in layer.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1 + 0.1 * torch.randn_like(p))
            else:
                p.normal_(0, 0.02)
    return layer


@pytest.mark.gpu
@pytest.mark.parametrize("varlen", [False, True])
@pytest.mark.parametrize("dh,partial", [(128, 0.25), (64, 1.0)])
def test_gated_attention_layer_matches_oracle(varlen, dh, partial):
    """The whole layer in bf16 (fused input projection, prologue, attention, o_proj) against the
    oracle's bf16 composition of the reference layer (softmax in fp32)."""
    layer = _layer(512, 8, 2, dh, partial, 1e6, seed=5).to(torch.bfloat16)
    b, t = (1, 300) if varlen else (2, 200)
    x = _randn(b, t, 512, seed=40)
    cu = torch.tensor([0, 17, 150, 300]) if varlen else None
    with torch.no_grad():
        out = layer.to(DEV)(x.to(DEV), None if cu is None else cu.to(DEV), None, cu).cpu()
    w = {n: p.detach().cpu() for n, p in layer.state_dict().items()}
    ref = gated_attention_layer(x, w, 8, 2, dh, layer.rotary.rot_dim, 1e6, cu_seqlens=cu)
    rel = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
    assert rel <= 2e-2, f"layer output relative L2 {rel:.3e}"
    assert_output_close(out, ref.float())


@pytest.mark.gpu
def test_gated_attention_layer_raises_on_grad():
    layer = _layer(256, 4, 2, 64, 0.25, 1e6, seed=6).to(DEV).to(torch.bfloat16)
    x = _randn(1, 16, 256, seed=1).to(DEV)
    with pytest.raises(NotImplementedError):
        layer(x)


@pytest.mark.gpu
def test_gated_attention_layer_fp32_stream_under_autocast():
    """The reference runs its mixers on the fp32 residual stream under autocast(bf16)
    (sore/train/trainer.py:175-176): fp32 parameters and fp32 x go in, the projections run in bf16 on
    the input cast to bf16, as nn.Linear's would. Checked against the oracle's bf16 composition."""
    layer = _layer(512, 8, 2, 128, 0.25, 1e6, seed=7)  # fp32 parameters
    g = torch.Generator().manual_seed(41)
    x = torch.randn(2, 160, 512, generator=g)  # fp32 activations
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = layer.to(DEV)(x.to(DEV)).float().cpu()
    w = {n: p.detach().cpu() for n, p in layer.state_dict().items()}
    ref = gated_attention_layer(x.to(torch.bfloat16), w, 8, 2, 128, layer.rotary.rot_dim, 1e6)
    rel = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
    assert rel <= 2e-2, f"layer output relative L2 {rel:.3e}"
    assert_output_close(out.to(torch.bfloat16), ref.float())
