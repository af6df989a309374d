"""GatedDeltaNet layer on the gfx950 ops: the reference layer with only its kernel imports swapped.

Counterpart of ``GatedDeltaNet`` in ``sore/model/gdn.py:81-209`` (its ``fla`` backend). The
reference's two caller flags keep their meaning and defaults (``sore/model/config.py:54-55``, both
False): ``gdn_fla_conv`` selects FLA's conv (fp32 weight, conv and SiLU in one rounding) over
``causal_conv1d_varlen(h, weight.to(h.dtype))`` followed by ``F.silu`` (the weight rounded to the
activation dtype, the conv output rounded before the SiLU, ``gdn.py:208-209``); ``fused_norm_gate``
selects ``rms_norm_gated`` (one rounding) over ``o_norm(o) * F.silu(gate)`` (the normalised ``o``
rounded before the product, ``gdn.py:180-188``). The presets the reference trains with set both
(``config.py:116,123``). The parameters, their names, shapes and init are the
reference's (``gdn.py:97-132``), so a reference ``state_dict`` loads unchanged; the forward keeps
the reference's call expressions (``gdn.py:145-189``) with ``chunk_gated_delta_rule``,
``causal_conv1d`` and ``rms_norm_gated`` taken from ``sorernn_amd`` instead of FLA. The chunk-index
patch of the FLA path (``gdn.py:31-78``) has no counterpart: the chunk kernel's grid depends only on
the number of sequences, so nothing is read back from the device.

The layer trains: the conv, the chunked rule and the gated norm are autograd functions over the
HIP backward kernels. With autograd off (inference), ``forward`` takes a fused route to the same
values: one GEMM for the q | k | v projections and one for a | b (weight concatenations cached
until a weight changes), then one ``qkv_causal_conv1d`` launch for the three convs + SiLU and the
q/k L2 norm, so the chunked rule runs without its in-kernel normalisation. Activations are bf16 (e.g. under ``torch.autocast("cuda",
dtype=torch.bfloat16)``, as the reference trains). The constructor reads only the ``ModelConfig``
fields ``GDNLayerConfig`` holds, so the reference's ``ModelConfig`` can be passed as is.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from sorernn_amd.ops import (causal_conv1d, chunk_gated_delta_rule, chunk_gated_delta_rule_gated_norm,
                             qkv_causal_conv1d, rms_norm_gated)
from sorernn_amd.ops import _plain_eager

_DT_MIN, _DT_MAX = 1e-3, 1e-1


@dataclass
class GDNLayerConfig:
    """The ``ModelConfig`` fields the layer reads (``sore/model/config.py:11,20-23,43,53-55``)."""

    d_model: int
    gdn_qk_heads: int = 1
    gdn_v_heads: int = 1
    gdn_head_dim: int = 128
    conv_kernel: int = 4
    norm_eps: float = 1e-6
    gdn_kernel_gate: bool = False
    gdn_fla_conv: bool = False
    fused_norm_gate: bool = False

    def __post_init__(self) -> None:
        if self.gdn_v_heads % self.gdn_qk_heads:
            raise ValueError(f"gdn_v_heads={self.gdn_v_heads} must be a multiple of gdn_qk_heads={self.gdn_qk_heads}")


class _NormWeight(nn.Module):
    """Holds ``o_norm.weight`` / ``o_norm.eps`` with the reference's names (``sore/model/layers.py:7-13``)."""

    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))


class GatedDeltaNet(nn.Module):
    """``o_proj(RMSNorm(o) * silu(g_proj(x)))`` with ``o`` from the chunked gated delta rule on gfx950.

    ``forward(x [B,T,D], cu_seqlens=None, cu_seqlens_cpu=None)``: with ``cu_seqlens`` (``[S+1]``,
    ``B == 1``) the conv and the recurrent state restart at every document; without it every batch
    row is one document. ``cu_seqlens_cpu`` (same values on the host) lets the ops validate the
    bounds without a device sync.
    """

    def __init__(self, cfg: GDNLayerConfig) -> None:
        super().__init__()
        self.kernel_gate = cfg.gdn_kernel_gate
        self.fla_conv = cfg.gdn_fla_conv
        self.fused_norm_gate = cfg.fused_norm_gate
        # inference route: True (the default) runs the gated RMSNorm in the chunk call
        # (chunk_gated_delta_rule_gated_norm: epilogue workgroups on the CUs the chains leave free,
        # or the norm kernel in place right after the chunk kernel); False calls the chunk op and the
        # norm kernel separately, as the reference's two calls do. Measured on one MI355X at the
        # config-4 GDN call (B=2, T=8192, H=16, d=128): 208 us against 186 + 45 us for the two
        # calls, the same output bit for bit; the layer forward 0.837 against 0.867 ms.
        self.fused_epilogue = True
        self.qk_heads = cfg.gdn_qk_heads
        self.v_heads = cfg.gdn_v_heads
        self.head_dim = cfg.gdn_head_dim
        d = cfg.d_model
        qk_dim = self.qk_heads * self.head_dim
        v_dim = self.v_heads * self.head_dim
        self.q_proj = nn.Linear(d, qk_dim, bias=False)
        self.k_proj = nn.Linear(d, qk_dim, bias=False)
        self.v_proj = nn.Linear(d, v_dim, bias=False)
        self.g_proj = nn.Linear(d, v_dim, bias=False)
        self.a_proj = nn.Linear(d, self.v_heads, bias=False)
        self.b_proj = nn.Linear(d, self.v_heads, bias=False)
        # depthwise conv weights [C, K] in fp32, nn.Conv1d's default init U(+-1/sqrt(K))
        bound = cfg.conv_kernel**-0.5
        self.conv_q = nn.Parameter(torch.empty(qk_dim, cfg.conv_kernel).uniform_(-bound, bound))
        self.conv_k = nn.Parameter(torch.empty(qk_dim, cfg.conv_kernel).uniform_(-bound, bound))
        self.conv_v = nn.Parameter(torch.empty(v_dim, cfg.conv_kernel).uniform_(-bound, bound))
        # decay: A ~ U(1, 16); dt log-uniform in [1e-3, 1e-1], dt_bias = softplus^-1(dt)
        self.A_log = nn.Parameter(torch.empty(self.v_heads).uniform_(1, 16).log())
        log_dt = torch.rand(self.v_heads) * (math.log(_DT_MAX) - math.log(_DT_MIN)) + math.log(_DT_MIN)
        dt = log_dt.exp()
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.o_norm = _NormWeight(self.head_dim, cfg.norm_eps)
        self.o_proj = nn.Linear(v_dim, d, bias=False)

    def _fused_weights(self, dtype: torch.dtype):
        key = tuple((w.data_ptr(), w._version) for w in (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
                                                          self.a_proj.weight, self.b_proj.weight, self.conv_q,
                                                          self.conv_k, self.conv_v)) + (dtype,)
        if key != getattr(self, "_fused_key", None):
            self._w_qkv = torch.cat([w.detach().to(dtype) for w in (self.q_proj.weight, self.k_proj.weight,
                                                                     self.v_proj.weight)], 0)
            self._w_ab = torch.cat([self.a_proj.weight.detach().to(dtype), self.b_proj.weight.detach().to(dtype)], 0)
            # the unfused conv rounds its weight to the activation dtype (sore/model/gdn.py:209)
            wc = torch.cat([self.conv_q.detach(), self.conv_k.detach(), self.conv_v.detach()], 0)
            self._w_conv = (wc if self.fla_conv else wc.to(dtype)).float()
            self._fused_key = key
        return self._w_qkv, self._w_ab, self._w_conv

    def _forward_fused(self, x: Tensor, cu_seqlens: Tensor | None, cu_seqlens_cpu: Tensor | None) -> Tensor:
        b, t, _ = x.shape
        hk, hv, dh = self.qk_heads, self.v_heads, self.head_dim
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else self.q_proj.weight.dtype
        w_qkv, w_ab, w_conv = self._fused_weights(dt)
        proj = F.linear(x, w_qkv)  # [B, T, q | k | v]
        q, k, v = qkv_causal_conv1d(proj, w_conv, hk * dh, hv * dh, dh, activation="silu", l2norm=True,
                                    cu_seqlens=cu_seqlens, cu_seqlens_cpu=cu_seqlens_cpu,
                                    round_before_activation=not self.fla_conv)
        ab = F.linear(x, w_ab)  # [B, T, a | b]
        a, bl = ab[..., :hv], ab[..., hv:]
        if self.kernel_gate:
            gate_kwargs = dict(use_gate_in_kernel=True, A_log=self.A_log, dt_bias=self.dt_bias,
                               use_beta_sigmoid_in_kernel=True)
            g, beta = a, bl
        else:
            gate_kwargs = {}
            g = -self.A_log.float().exp() * F.softplus(a.float() + self.dt_bias.float())
            beta = bl.sigmoid()
        gate = self.g_proj(x).view(b, t, hv, dh)
        if self.fused_epilogue and q.dtype == torch.bfloat16 and _plain_eager(q):
            # the gated RMSNorm in the chunk call: y is written over the stored o
            o, _ = chunk_gated_delta_rule_gated_norm(
                q.view(b, t, hk, dh), k.view(b, t, hk, dh), v.view(b, t, hv, dh), g, beta, gate,
                self.o_norm.weight, self.o_norm.eps, norm_split=not self.fused_norm_gate, scale=dh**-0.5,
                cu_seqlens=cu_seqlens, cu_seqlens_cpu=cu_seqlens_cpu, **gate_kwargs,
            )
            return self.o_proj(o.flatten(-2))
        o, _ = chunk_gated_delta_rule(
            q.view(b, t, hk, dh), k.view(b, t, hk, dh), v.view(b, t, hv, dh), g, beta, scale=dh**-0.5,
            cu_seqlens=cu_seqlens, cu_seqlens_cpu=cu_seqlens_cpu, **gate_kwargs,
        )
        return self.o_proj(self._norm_gate(o, gate).flatten(-2))

    def _norm_gate(self, o: Tensor, gate: Tensor) -> Tensor:
        if self.fused_norm_gate:
            # RMSNorm(o) * silu(gate) in one kernel, fp32 math, one rounding (sore/model/gdn.py:182-186)
            return rms_norm_gated(o, gate, self.o_norm.weight, None, activation="swish", eps=self.o_norm.eps)
        # o_norm(o) rounded to o's dtype, then times silu(gate) (sore/model/gdn.py:188)
        return rms_norm_gated(o, None, self.o_norm.weight, None, eps=self.o_norm.eps) * F.silu(gate)

    def forward(self, x: Tensor, cu_seqlens: Tensor | None = None, cu_seqlens_cpu: Tensor | None = None) -> Tensor:
        if not torch.is_grad_enabled() and self.head_dim in (64, 128):
            dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else self.q_proj.weight.dtype
            if dt in (torch.bfloat16, torch.float16):
                return self._forward_fused(x, cu_seqlens, cu_seqlens_cpu)
        return self._forward_reference(x, cu_seqlens, cu_seqlens_cpu)

    def _forward_reference(self, x: Tensor, cu_seqlens: Tensor | None = None,
                           cu_seqlens_cpu: Tensor | None = None) -> Tensor:
        b, t, _ = x.shape

        def conv(h: Tensor, weight: Tensor) -> Tensor:
            if self.fla_conv:
                return causal_conv1d(h, weight, activation="silu", cu_seqlens=cu_seqlens,
                                     cu_seqlens_cpu=cu_seqlens_cpu)[0]
            # the weight rounded to the activation dtype, the conv output rounded before the SiLU
            # (sore/model/gdn.py:208-209)
            return F.silu(causal_conv1d(h, weight.to(h.dtype), activation=None, cu_seqlens=cu_seqlens,
                                        cu_seqlens_cpu=cu_seqlens_cpu)[0])

        q = conv(self.q_proj(x), self.conv_q).view(b, t, self.qk_heads, self.head_dim)
        k = conv(self.k_proj(x), self.conv_k).view(b, t, self.qk_heads, self.head_dim)
        v = conv(self.v_proj(x), self.conv_v).view(b, t, self.v_heads, self.head_dim)
        scale = self.head_dim**-0.5
        if self.kernel_gate:
            gate_kwargs = dict(use_gate_in_kernel=True, A_log=self.A_log, dt_bias=self.dt_bias,
                               use_beta_sigmoid_in_kernel=True)
            g, beta = self.a_proj(x), self.b_proj(x)
        else:
            gate_kwargs = {}
            g, beta = self._gate_and_beta(x)
        o, _ = chunk_gated_delta_rule(
            q, k, v, g, beta, scale=scale, cu_seqlens=cu_seqlens, cu_seqlens_cpu=cu_seqlens_cpu,
            use_qk_l2norm_in_kernel=True, **gate_kwargs,
        )
        gate = self.g_proj(x).view(b, t, self.v_heads, self.head_dim)
        return self.o_proj(self._norm_gate(o, gate).flatten(-2))

    def _gate_and_beta(self, x: Tensor) -> tuple[Tensor, Tensor]:
        # g (log-decay, <= 0) in fp32; beta may stay in the activation dtype (sore/model/gdn.py:191-194)
        g = -self.A_log.float().exp() * F.softplus(self.a_proj(x).float() + self.dt_bias.float())
        return g, self.b_proj(x).sigmoid()
