"""CPU restatement of soreRNN's gated global attention layer (the parity oracle of the block pair).

TEST INFRASTRUCTURE ONLY, like ``oracle/gdn_oracle.py``: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it. The product package never imports it.

Restated (read, never imported) from ToGoodForReal/soreRNN:
- ``partial_rotary``: ``PartialRotary`` (``sore/model/rope.py:6-41``), the same fp32 frequency math
  and the same casts to the activation dtype before the bf16 tensor arithmetic;
- ``causal_attention``: ``GatedAttention._sdpa`` (``sore/model/attention.py:124-135``), written
  out as scores, mask, softmax and weighted sum in ``promote(dtype, float32)`` (fp64 stays fp64),
  with GQA as ``repeat_interleave`` (``enable_gqa=True``);
- ``gated_attention_layer``: ``GatedAttention.forward`` (``attention.py:98-122``) on a dict of the
  layer's weights.

Pinning (``tests/test_attention_oracle.py``): ``causal_attention`` against
``F.scaled_dot_product_attention`` (a library routine) with ``is_causal`` and with the dense
document mask, and against per-document runs; ``partial_rotary`` against the rotation's closed
forms (position 0 is the identity, each rotated pair keeps its norm, q.k after rotation depends only
on the position difference, dims past ``rot_dim`` pass unchanged) and a planted sign error;
``gated_attention_layer`` against a composition of the pinned parts with the reference's layout.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from oracle.gdn_oracle import doc_ids_from_cu_seqlens, positions_from_cu_seqlens, rms_norm

__all__ = ["causal_attention", "gated_attention_layer", "partial_rotary", "rotary_cos_sin"]


def rotary_cos_sin(positions: Tensor, rot_dim: int, theta: float, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    """``cos, sin [T, rot_dim]`` in ``dtype`` (``sore/model/rope.py:29-34``: fp32 until the cast)."""
    exponent = torch.arange(0, rot_dim, 2, dtype=torch.float32) / rot_dim
    inv_freq = 1.0 / theta**exponent
    freqs = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def partial_rotary(x: Tensor, positions: Tensor, rot_dim: int, theta: float) -> Tensor:
    """GPT-NeoX ``rotate_half`` rotary on the first ``rot_dim`` dims of ``x [B,T,H,D]`` (``rope.py:36-40``).

    The products and the sum run in ``x.dtype`` tensor arithmetic (each rounded to ``x.dtype``), as
    the reference's ``x_rot * cos + rotated * sin`` does.
    """
    if rot_dim <= 0 or rot_dim % 2 or rot_dim > x.shape[-1]:
        raise ValueError(f"rot_dim={rot_dim} must be even, positive and <= head_dim")
    cos, sin = rotary_cos_sin(positions, rot_dim, theta, x.dtype)
    cos, sin = cos[None, :, None, :], sin[None, :, None, :]
    half = rot_dim // 2
    x_rot, x_pass = x[..., :rot_dim], x[..., rot_dim:]
    rotated = torch.cat((-x_rot[..., half:], x_rot[..., :half]), dim=-1)
    return torch.cat((x_rot * cos + rotated * sin, x_pass), dim=-1)


def causal_attention(q: Tensor, k: Tensor, v: Tensor, doc_ids: Tensor | None = None, scale: float | None = None) -> Tensor:
    """Causal GQA attention, ``q [B,HQ,T,D]``, ``k, v [B,HKV,T,D]`` -> ``[B,HQ,T,D]`` in ``q.dtype``.

    ``doc_ids [T]`` restricts each query to keys of its own document (``attention.py:130-135``).
    Math in ``promote(q.dtype, float32)``.
    """
    cdt = torch.promote_types(q.dtype, torch.float32)
    hq, hkv = q.shape[1], k.shape[1]
    qf, kf, vf = q.to(cdt), k.to(cdt).repeat_interleave(hq // hkv, dim=1), v.to(cdt).repeat_interleave(hq // hkv, dim=1)
    t = q.shape[2]
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    s = (qf @ kf.transpose(-1, -2)) * scale
    allowed = torch.ones(t, t, dtype=torch.bool).tril()
    if doc_ids is not None:
        allowed = allowed & (doc_ids[:, None] == doc_ids[None, :])
    s = s.masked_fill(~allowed, float("-inf"))
    return (torch.softmax(s, dim=-1) @ vf).to(q.dtype)


def gated_attention_layer(x: Tensor, w: dict, heads: int, kv_heads: int, head_dim: int, rot_dim: int, theta: float,
                          eps: float = 1e-6, cu_seqlens: Tensor | None = None, attn_dtype: torch.dtype | None = None):
    """``GatedAttention.forward`` (``attention.py:98-122``) on weights ``w`` (the layer's state_dict keys).

    Every intermediate is held in ``x.dtype`` as in the reference's bf16 run; ``attn_dtype``
    (default: promote(x.dtype, fp32)) is the precision of the softmax and the weighted sum.
    """
    b, t, _ = x.shape
    lin = lambda a, name: a @ w[name].to(a.dtype).T  # noqa: E731
    q = rms_norm(lin(x, "q_proj.weight").view(b, t, heads, head_dim), w["q_norm.weight"], eps)
    k = rms_norm(lin(x, "k_proj.weight").view(b, t, kv_heads, head_dim), w["k_norm.weight"], eps)
    v = lin(x, "v_proj.weight").view(b, t, kv_heads, head_dim)
    if cu_seqlens is None:
        doc_ids, positions = None, torch.arange(t)
    else:
        doc_ids, positions = doc_ids_from_cu_seqlens(cu_seqlens, t), positions_from_cu_seqlens(cu_seqlens, t)
    q, k = partial_rotary(q, positions, rot_dim, theta), partial_rotary(k, positions, rot_dim, theta)
    adt = attn_dtype or torch.promote_types(x.dtype, torch.float32)
    o = causal_attention(q.transpose(1, 2).to(adt), k.transpose(1, 2).to(adt), v.transpose(1, 2).to(adt), doc_ids)
    o = o.to(x.dtype).transpose(1, 2).reshape(b, t, heads * head_dim)
    return lin(o * torch.sigmoid(lin(x, "gate_proj.weight")), "o_proj.weight")
