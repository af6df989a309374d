"""Gated global attention layer on the gfx950 kernels: the attention half of the hybrid block pair.

Counterpart of ``GatedAttention`` in ``sore/model/attention.py:60-135``: causal GQA attention with
q/k RMSNorm, partial rotary embedding (GPT-NeoX ``rotate_half`` on the first
``int(head_dim * rope_partial)`` dims, ``sore/model/rope.py``) and a sigmoid output gate,
``o_proj(attn * sigmoid(gate_proj(x)))``. The parameters keep the reference's names, shapes and
bias-free projections (``attention.py:83-91``), so a reference ``state_dict`` loads unchanged.

Work per forward:
- one GEMM for the four input projections (q | gate | k | v weights concatenated; the
  concatenation is cached until a weight changes), a library GEMM (hipBLASLt through torch);
- ``gdn_attn_qk_norm_rope_fwd``: RMSNorm of q and k per head plus the rotary embedding, reading the
  column slices of the projection output in place;
- ``gdn_attn_fwd``: causal (document-causal with ``cu_seqlens``) GQA flash attention with the
  sigmoid gate applied on the way out;
- the output projection (library GEMM).

Forward only: a call whose inputs or parameters require grad raises ``NotImplementedError``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from sorernn_amd import _lib
from sorernn_amd.ops import _check_cuda, _cu_info, _no_grad_check

__all__ = ["AttnLayerConfig", "GatedAttention", "attn_qk_norm_rope", "gated_attention"]


def _row_view_ok(x: Tensor, width: int) -> int:
    """Row stride (elements) of a [B, T, >= width] view whose last axis is contiguous."""
    if x.dim() != 3 or x.stride(2) != 1 or x.shape[2] != width:
        raise ValueError(f"expected a [B, T, {width}] tensor with a contiguous last axis, got {tuple(x.shape)} "
                         f"strides {x.stride()}")
    b, t = x.shape[:2]
    if t > 1 and b > 1 and x.stride(0) != t * x.stride(1):
        raise ValueError("rows of the batch must be evenly strided (a [B*T, width] view)")
    if x.data_ptr() % 16:
        raise ValueError("tensor data must be 16-byte aligned")
    return x.stride(1) if t > 1 else (x.stride(0) if b > 1 else width)


def attn_qk_norm_rope(q_in: Tensor, k_in: Tensor, q_weight: Tensor, k_weight: Tensor, heads: int, kv_heads: int,
                      rot_dim: int, theta: float, eps: float = 1e-6, cu_seqlens: Tensor | None = None,
                      cu_seqlens_cpu: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """RMSNorm of every q/k head row followed by the rotary embedding (``attention.py:105-116``).

    ``q_in [B,T,heads*D]`` and ``k_in [B,T,kv_heads*D]`` (bf16; views with a row stride are read in
    place); weights ``[D]``. Positions are the token index, restarting at 0 in every document with
    ``cu_seqlens`` (``sore/model/varlen.py:17-21``). Returns contiguous ``q [B,T,heads,D]`` and
    ``k [B,T,kv_heads,D]``.
    """
    name = "attn_qk_norm_rope"
    _check_cuda(name, q_in, k_in, q_weight, k_weight, cu_seqlens)
    _no_grad_check(name, q_in, k_in, q_weight, k_weight)
    if q_in.dtype != torch.bfloat16 or k_in.dtype != torch.bfloat16:
        raise NotImplementedError(f"{name}: bf16 activations only, got {q_in.dtype}/{k_in.dtype}")
    b, t = q_in.shape[:2]
    d = q_weight.numel()
    if k_weight.numel() != d or q_in.shape[-1] != heads * d or k_in.shape[-1] != kv_heads * d or k_in.shape[:2] != (b, t):
        raise ValueError(f"{name}: shapes q {tuple(q_in.shape)}, k {tuple(k_in.shape)}, weights {d} do not match "
                         f"heads={heads}, kv_heads={kv_heads}")
    qs, ks = _row_view_ok(q_in, heads * d), _row_view_ok(k_in, kv_heads * d)
    n, flags = _cu_info(name, cu_seqlens, cu_seqlens_cpu, b, t)
    w_dtype = q_weight.dtype if q_weight.dtype in (torch.float32, torch.bfloat16) else torch.float32
    qw, kw = q_weight.detach().to(w_dtype).contiguous(), k_weight.detach().to(w_dtype).contiguous()
    q = torch.empty(b, t, heads, d, device=q_in.device, dtype=torch.bfloat16)
    k = torch.empty(b, t, kv_heads, d, device=q_in.device, dtype=torch.bfloat16)
    _lib.call("gdn_attn_qk_norm_rope_fwd", q_in.data_ptr(), qs, k_in.data_ptr(), ks, qw.data_ptr(), kw.data_ptr(),
              _lib.dtype_code(w_dtype), q.data_ptr(), k.data_ptr(), _lib.ptr(cu_seqlens), b, t, heads, kv_heads, d, n,
              int(rot_dim), float(theta), float(eps), flags, _lib.stream_of(q_in))
    return q, k


def gated_attention(q: Tensor, k: Tensor, v: Tensor, gate: Tensor, cu_seqlens: Tensor | None = None,
                    cu_seqlens_cpu: Tensor | None = None, scale: float | None = None) -> Tensor:
    """``softmax(scale q k^T + mask) v * sigmoid(gate)`` (``attention.py:122-135``), bf16.

    ``q [B,T,HQ,D]``, ``k [B,T,HKV,D]`` contiguous; ``v [B,T,HKV*D]`` and ``gate [B,T,HQ*D]`` may
    be column slices of a wider projection output. Causal per batch row, or per document with
    ``cu_seqlens`` (``B == 1``). ``scale`` defaults to ``D**-0.5`` (SDPA's default). Returns
    ``o [B,T,HQ*D]``.
    """
    name = "gated_attention"
    _check_cuda(name, q, k, v, gate, cu_seqlens)
    _no_grad_check(name, q, k, v, gate)
    if q.dim() != 4 or k.dim() != 4 or k.shape[:2] != q.shape[:2] or k.shape[3] != q.shape[3]:
        raise ValueError(f"{name}: expected q [B,T,HQ,D] and k [B,T,HKV,D], got {tuple(q.shape)}, {tuple(k.shape)}")
    b, t, hq, d = q.shape
    hkv = k.shape[2]
    if hq % hkv:
        raise ValueError(f"{name}: q heads ({hq}) must be a multiple of kv heads ({hkv})")
    if any(x.dtype != torch.bfloat16 for x in (q, k, v, gate)):
        raise NotImplementedError(f"{name}: bf16 only")
    if not (q.is_contiguous() and k.is_contiguous()):
        raise ValueError(f"{name}: q and k must be contiguous")
    vs, gs = _row_view_ok(v, hkv * d), _row_view_ok(gate, hq * d)
    if v.shape[:2] != (b, t) or gate.shape[:2] != (b, t):
        raise ValueError(f"{name}: v / gate must be [B, T, *] with B={b}, T={t}")
    n, flags = _cu_info(name, cu_seqlens, cu_seqlens_cpu, b, t)
    o = torch.empty(b, t, hq * d, device=q.device, dtype=torch.bfloat16)
    _lib.call("gdn_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), vs, gate.data_ptr(), gs, o.data_ptr(),
              _lib.ptr(cu_seqlens), b, t, hq, hkv, d, n, float(d**-0.5 if scale is None else scale), flags,
              _lib.stream_of(q))
    return o


@dataclass
class AttnLayerConfig:
    """The ``ModelConfig`` fields the layer reads (``sore/model/config.py:11,25-30,43``)."""

    d_model: int
    attn_heads: int = 1
    attn_kv_heads: int = 1
    attn_head_dim: int = 128
    rope_theta: float = 1e7
    rope_partial: float = 0.25
    norm_eps: float = 1e-6

    def __post_init__(self) -> None:
        if self.attn_heads % self.attn_kv_heads:
            raise ValueError(f"attn_heads={self.attn_heads} must be a multiple of attn_kv_heads={self.attn_kv_heads}")


class _RMSNormWeight(nn.Module):
    """``weight`` [dim] and ``eps`` under the reference's names (``sore/model/layers.py:7-13``)."""

    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))


class _Rotary(nn.Module):
    """Partial rotary settings (``sore/model/rope.py:6-22``): no parameters, the same validation."""

    def __init__(self, head_dim: int, partial: float, theta: float) -> None:
        super().__init__()
        rot_dim = int(head_dim * partial)
        if rot_dim <= 0 or rot_dim % 2 != 0 or rot_dim > head_dim:
            raise ValueError(f"rot_dim=int({head_dim} * {partial})={rot_dim} must be even, positive and <= head_dim")
        self.head_dim, self.rot_dim, self.theta = head_dim, rot_dim, theta


class GatedAttention(nn.Module):
    """``o_proj(attn * sigmoid(gate_proj(x)))`` with causal GQA attention and partial RoPE on gfx950.

    ``forward(x [B,T,D], cu_seqlens=None, block_mask=None, cu_seqlens_cpu=None)``: with
    ``cu_seqlens`` (``[S+1]``, ``B == 1``) attention is causal inside each document and the rotary
    positions restart at 0 in each; without it every batch row is one document. ``block_mask`` (the
    reference's flex ``BlockMask``) is accepted and not needed: the kernel applies the
    document-causal mask itself.
    """

    def __init__(self, cfg: AttnLayerConfig) -> None:
        super().__init__()
        self.heads = cfg.attn_heads
        self.kv_heads = cfg.attn_kv_heads
        self.head_dim = cfg.attn_head_dim
        d = cfg.d_model
        self.q_proj = nn.Linear(d, self.heads * self.head_dim, bias=False)
        self.gate_proj = nn.Linear(d, self.heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(d, self.kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(d, self.kv_heads * self.head_dim, bias=False)
        self.q_norm = _RMSNormWeight(self.head_dim, cfg.norm_eps)
        self.k_norm = _RMSNormWeight(self.head_dim, cfg.norm_eps)
        self.rotary = _Rotary(self.head_dim, cfg.rope_partial, cfg.rope_theta)
        self.o_proj = nn.Linear(self.heads * self.head_dim, d, bias=False)
        self._wcat_key = None
        self._wcat = None

    def _fused_weight(self, dtype: torch.dtype) -> Tensor:
        ws = (self.q_proj.weight, self.gate_proj.weight, self.k_proj.weight, self.v_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws) + (dtype,)
        if key != self._wcat_key:
            self._wcat = torch.cat([w.detach().to(dtype) for w in ws], dim=0)
            self._wcat_key = key
        return self._wcat

    def forward(self, x: Tensor, cu_seqlens: Tensor | None = None, block_mask=None,
                cu_seqlens_cpu: Tensor | None = None) -> Tensor:
        b, t, _ = x.shape
        if cu_seqlens is not None and b != 1:
            raise ValueError(f"cu_seqlens requires B == 1 (packed [1, N] layout); got B={b}")
        _no_grad_check("GatedAttention", x, *self.parameters())
        hq, hkv, dh = self.heads, self.kv_heads, self.head_dim
        # under autocast the projections run in the autocast dtype with the input cast to it, as
        # nn.Linear's would (the reference feeds its fp32 residual stream into the mixers under
        # autocast); without autocast the input is cast to the weights' dtype
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else self.q_proj.weight.dtype
        if dt not in (torch.bfloat16, torch.float16):
            raise NotImplementedError(f"GatedAttention: the gfx950 kernels take bf16/fp16 activations, got {dt}")
        proj = F.linear(x.to(dt), self._fused_weight(dt))  # [B, T, q | gate | k | v]
        nq, nkv = hq * dh, hkv * dh
        q_in, gate = proj[..., :nq], proj[..., nq:2 * nq]
        k_in, v = proj[..., 2 * nq:2 * nq + nkv], proj[..., 2 * nq + nkv:]
        q, k = attn_qk_norm_rope(q_in, k_in, self.q_norm.weight, self.k_norm.weight, hq, hkv, self.rotary.rot_dim,
                                 self.rotary.theta, self.q_norm.eps, cu_seqlens, cu_seqlens_cpu)
        o = gated_attention(q, k, v, gate, cu_seqlens, cu_seqlens_cpu)
        return self.o_proj(o)
