"""Seeded synthetic inputs for the benchmark configurations of the GDN path.

All draws use a CPU ``torch.Generator`` seeded with ``1000 + config index`` (so the CPU baseline and
the GPU run see bit-identical inputs) in the order q, k, v, beta-logit, g-normal, g-uniform, h0:

- q, k ~ N(0,1) in fp32, L2-normalised per (token, head), then cast;
- v ~ N(0,1);
- beta = sigmoid(N(0,1));
- g = -softplus(N(0,1)) * exp(U(-4,-1))  (per-token log-decay);
- h0 ~ N(0, 0.02) fp32.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

# BASELINE configs 0-3 (config 4, the full block pair, is outside the token-mixing path)
CONFIGS = {
    0: dict(B=1, T=256, H=4, K=64, dtype=torch.float32, h0=False),
    1: dict(B=4, T=4096, H=16, K=128, dtype=torch.bfloat16, h0=True),
    3: dict(B=1, T=32768, H=16, K=128, dtype=torch.bfloat16, h0=True, n_docs=8),
}


@dataclass
class GDNInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    h0: torch.Tensor | None
    cu_seqlens: torch.Tensor | None
    scale: float

    def to(self, device) -> "GDNInputs":
        mv = lambda x: None if x is None else x.to(device)  # noqa: E731
        return GDNInputs(mv(self.q), mv(self.k), mv(self.v), mv(self.g), mv(self.beta), mv(self.h0),
                         mv(self.cu_seqlens), self.scale)


def gdn_inputs(B, T, H, K, V=None, HV=None, dtype=torch.bfloat16, seed=1000, h0=False, n_states=None,
               cu_seqlens=None) -> GDNInputs:
    V = K if V is None else V
    HV = H if HV is None else HV
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, K, generator=gen), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, T, H, K, generator=gen), dim=-1).to(dtype)
    v = torch.randn(B, T, HV, V, generator=gen).to(dtype)
    beta = torch.randn(B, T, HV, generator=gen).sigmoid()
    g = -F.softplus(torch.randn(B, T, HV, generator=gen)) * (torch.rand(B, T, HV, generator=gen) * 3 - 4).exp()
    n = n_states if n_states is not None else (B if cu_seqlens is None else cu_seqlens.numel() - 1)
    s0 = 0.02 * torch.randn(n, HV, K, V, generator=gen) if h0 else None
    return GDNInputs(q, k, v, g, beta, s0, cu_seqlens, K**-0.5)


def varlen_cu_seqlens(n_docs: int, total: int, lo: int, hi: int, seed: int) -> torch.Tensor:
    """Document lengths ~U[lo, hi] (integers, seeded), rescaled to sum exactly ``total``.

    The rounding remainder goes to the last document.
    """
    gen = torch.Generator().manual_seed(seed)
    raw = torch.randint(lo, hi + 1, (n_docs,), generator=gen).double()
    lens = torch.floor(raw * total / raw.sum()).long().clamp_min(1)
    lens[-1] += total - int(lens.sum())
    return torch.cat([torch.zeros(1, dtype=torch.long), lens.cumsum(0)])


def config_inputs(index: int) -> GDNInputs:
    """Inputs of BASELINE config 0, 1 or 3 (on the CPU)."""
    c = CONFIGS[index]
    seed = 1000 + index
    if index == 3:
        cu = varlen_cu_seqlens(c["n_docs"], c["T"], 512, 8192, seed)
        return gdn_inputs(c["B"], c["T"], c["H"], c["K"], dtype=c["dtype"], seed=seed, h0=c["h0"], cu_seqlens=cu)
    return gdn_inputs(c["B"], c["T"], c["H"], c["K"], dtype=c["dtype"], seed=seed, h0=c["h0"])


@dataclass
class DecodeInputs:
    x_qkv: torch.Tensor
    conv_state: torch.Tensor
    conv_weight: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    state: torch.Tensor
    H: int
    HV: int
    D: int


def decode_inputs(B=64, H=16, HV=16, D=128, W=4, dtype=torch.bfloat16, seed=1002) -> DecodeInputs:
    """one token of pre-conv q|k|v per sequence, a width-W conv cache, fp32 state.

    g and beta are distributed as in config 0; the state ~ N(0, 0.02); the conv weight follows the
    layer's init U(+-1/sqrt(W)) (``sore/model/gdn.py:120-123``); the cache holds N(0,1) inputs.
    """
    gen = torch.Generator().manual_seed(seed)
    c = (2 * H + HV) * D
    x = torch.randn(B, c, generator=gen).to(dtype)
    conv_state = torch.randn(B, c, W, generator=gen).to(dtype)
    bound = W**-0.5
    conv_weight = (torch.rand(c, W, generator=gen) * 2 - 1) * bound
    beta = torch.randn(B, HV, generator=gen).sigmoid()
    g = -F.softplus(torch.randn(B, HV, generator=gen)) * (torch.rand(B, HV, generator=gen) * 3 - 4).exp()
    state = 0.02 * torch.randn(B, HV, D, D, generator=gen)
    return DecodeInputs(x, conv_state, conv_weight, g, beta, state, H, HV, D)
