"""CPU restatement of soreRNN's Gated DeltaNet token-mixing path (the parity oracle).

TEST INFRASTRUCTURE ONLY. This module is the checker for the HIP kernels and the timed CPU baseline
of ``bench.py``. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it. The product package ``sorernn_amd`` never imports it and has no CPU fallback.

Every function restates a reference function in plain torch CPU code written for this build. The
reference is read, never imported. Citations are ``file:line`` in ToGoodForReal/soreRNN.

Pinning (each function is checked against something other than its own formula; see
``tests/test_oracle.py``):

- ``recurrent_gated_delta_rule`` / ``naive_gated_delta_rule``: the reference's known-answer tests
  (T=1 closed form, two hand-computed steps, varlen == separate, state reset, single-token documents,
  B==1 and coverage errors, low-precision dtype), an independent matrix-transition formulation, the
  closed form of one step from a non-zero state, split invariance (which pins ``initial_state`` and
  the final state), and brute force on tiny inputs.
- ``chunk_gated_delta_rule_ref``: equal to the recurrence in fp64 (1e-10) on config-0 shapes,
  including partial chunks, varlen and initial states.
- ``matrix_transition_rule``: equal to the delta form, and to explicit products of 2x2 matrices.
- ``causal_conv1d_varlen``: ``F.conv1d`` for K in {1,2,4}, the impulse known answer
  ``[0,0,100,10,1]``, no cross-document leak, NaN isolation.
- ``doc_ids_from_cu_seqlens`` / ``positions_from_cu_seqlens``: the reference's known id/position lists.
- ``l2norm``: ``F.normalize``. ``rms_norm``: the formula in the reference test. ``rms_norm_gated``:
  ``rms_norm(x) * silu(gate)`` in fp64.
- ``gate_and_beta``: the closed form for a==-dt_bias (softplus(0)=log 2) and ``F.softplus``.
- ``decode_step_ref``: equal to the last token of the full-sequence conv + recurrence.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

__all__ = [
    "causal_conv1d_silu",
    "causal_conv1d_varlen",
    "chunk_gated_delta_rule_bwd_ref",
    "chunk_gated_delta_rule_ref",
    "conv_state_from_sequence",
    "decode_step_ref",
    "doc_ids_from_cu_seqlens",
    "gate_and_beta",
    "gva_expand",
    "l2norm",
    "matrix_transition_rule",
    "naive_gated_delta_rule",
    "positions_from_cu_seqlens",
    "recurrent_gated_delta_rule",
    "rms_norm",
    "rms_norm_gated",
]


# --------------------------------------------------------------------------------------------------
# varlen helpers  (sore/model/varlen.py:10-21)
# --------------------------------------------------------------------------------------------------
def doc_ids_from_cu_seqlens(cu_seqlens: Tensor, n: int) -> Tensor:
    """Document id of each packed position, as ``LongTensor[n]``.

    Follows ``sore/model/varlen.py:10-14``: a position equal to a boundary belongs to the next
    document (``searchsorted(..., right=True)`` over the interior and final boundaries).
    """
    positions = torch.arange(n, device=cu_seqlens.device, dtype=cu_seqlens.dtype)
    return torch.searchsorted(cu_seqlens[1:].contiguous(), positions, right=True).long()


def positions_from_cu_seqlens(cu_seqlens: Tensor, n: int) -> Tensor:
    """Position of each token inside its document (``sore/model/varlen.py:17-21``)."""
    ids = doc_ids_from_cu_seqlens(cu_seqlens, n)
    return torch.arange(n, device=cu_seqlens.device, dtype=torch.long) - cu_seqlens.long()[ids]


# --------------------------------------------------------------------------------------------------
# gated delta rule, sequential form  (sore/model/gdn_ref.py:11-61)
# --------------------------------------------------------------------------------------------------
def gva_expand(x: Tensor, n_v_heads: int) -> Tensor:
    """Repeat q/k heads for grouped value heads: v-head i reads q/k head ``i // rep``.

    ``sore/model/gdn.py:171-174`` (``repeat_interleave`` over the head axis, consecutive grouping).
    """
    h = x.shape[2]
    if n_v_heads == h:
        return x
    if n_v_heads % h:
        raise ValueError(f"v heads ({n_v_heads}) must be a multiple of q/k heads ({h})")
    return x.repeat_interleave(n_v_heads // h, dim=2)


def _recurrence(q, k, v, g, beta, scale, state):
    """One contiguous segment; ``state [B,H,K,V]`` is the state before the first token.

    Same per-token order as ``sore/model/gdn_ref.py:17-21``: decay, delta, rank-1 write, read.
    Returns ``(o [B,T,H,V], final state)``.
    """
    outputs = []
    for i in range(q.shape[1]):
        state = state * g[:, i].exp()[..., None, None]
        delta = (v[:, i] - (state * k[:, i, ..., None]).sum(-2)) * beta[:, i, ..., None]
        state = state + k[:, i, ..., None] * delta[..., None, :]
        outputs.append(torch.einsum("bhd,bhdm->bhm", q[:, i] * scale, state))
    if outputs:
        return torch.stack(outputs, dim=1), state
    return q.new_zeros(q.shape[0], 0, q.shape[2], v.shape[-1]), state


def _check_cu(cu_seqlens: Tensor, batch: int, t: int) -> list[int]:
    # sore/model/gdn_ref.py:42-43 and :52-55 (same error wording as the reference's tests match on)
    if batch != 1:
        raise ValueError(f"cu_seqlens requires B == 1, got B = {batch}")
    bounds = [int(x) for x in cu_seqlens.tolist()]
    if bounds[0] != 0 or bounds[-1] != t:
        raise ValueError(f"cu_seqlens must go from 0 to T = {t}, got {bounds[0]}..{bounds[-1]}")
    return bounds


def recurrent_gated_delta_rule(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    scale: float | None = None,
    initial_state: Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: Tensor | None = None,
):
    """Sequential gated delta rule with an initial state and an optional final state.

    Restates ``naive_gated_delta_rule`` (``sore/model/gdn_ref.py:25-61``) and extends it with
    ``initial_state [N,HV,K,V]`` and a final-state output, which the reference does not have.
    Layouts: ``q,k [B,T,H,K]``, ``v [B,T,HV,V]``, ``g,beta [B,T,HV]``; ``N = B``, or the number of
    documents with ``cu_seqlens`` (then ``B == 1``). Computes in ``promote(v.dtype, float32)``
    (``gdn_ref.py:45-47``), so fp64 stays fp64. Returns ``o`` in ``v.dtype`` and the final state in
    the compute dtype (or ``None``).
    """
    b, t, _, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    if scale is None:
        scale = kd**-0.5
    out_dtype = v.dtype
    cdt = torch.promote_types(out_dtype, torch.float32)
    q, k = gva_expand(q, hv), gva_expand(k, hv)
    q, k, v, g, beta = (x.to(cdt) for x in (q, k, v, g, beta))

    if cu_seqlens is None:
        state = q.new_zeros(b, hv, kd, vd) if initial_state is None else initial_state.to(cdt).clone()
        o, state = _recurrence(q, k, v, g, beta, scale, state)
        return o.to(out_dtype), (state if output_final_state else None)

    bounds = _check_cu(cu_seqlens, b, t)
    outs, finals = [], []
    for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        if initial_state is None:
            s0 = q.new_zeros(1, hv, kd, vd)
        else:
            s0 = initial_state[n : n + 1].to(cdt).clone()
        o, s = _recurrence(q[:, a:e], k[:, a:e], v[:, a:e], g[:, a:e], beta[:, a:e], scale, s0)
        outs.append(o)
        finals.append(s)
    o = torch.cat(outs, dim=1).to(out_dtype)
    return o, (torch.cat(finals, dim=0) if output_final_state else None)


def naive_gated_delta_rule(q, k, v, g, beta, scale, cu_seqlens=None):
    """The reference oracle's exact interface (``sore/model/gdn_ref.py:25-33``): returns only ``o``."""
    return recurrent_gated_delta_rule(q, k, v, g, beta, scale, cu_seqlens=cu_seqlens)[0]


def matrix_transition_rule(q, k, v, g, beta, scale, initial_state=None):
    """Independent formulation: ``S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T``, ``o_t = S_t q_t``.

    The state here is ``[V,K]`` as written in ``docs/superpowers/specs/2026-10-23-sorernn-v2-design.md:38-43``
    (the transpose of ``gdn_ref.py``'s ``[K,V]``); ``a_t = exp(g_t)``. fp64, no varlen. Returns
    ``(o [B,T,H,V], final state [B,H,K,V])``.
    """
    q, k, v, g, beta = (x.double() for x in (q, k, v, g, beta))
    b, t, h, kd = q.shape
    vd = v.shape[-1]
    eye = torch.eye(kd, dtype=torch.float64)
    s = torch.zeros(b, h, vd, kd, dtype=torch.float64) if initial_state is None else initial_state.double().transpose(-1, -2).clone()
    outs = []
    for i in range(t):
        kk = k[:, i]
        trans = eye - beta[:, i, :, None, None] * kk[..., :, None] * kk[..., None, :]
        s = g[:, i].exp()[..., None, None] * (s @ trans) + beta[:, i, :, None, None] * v[:, i, ..., :, None] * kk[..., None, :]
        outs.append(scale * (s @ q[:, i, ..., None])[..., 0])
    return torch.stack(outs, dim=1), s.transpose(-1, -2)


# --------------------------------------------------------------------------------------------------
# chunked (UT / WY) formulation, fp64 -- the algebra the HIP prefill kernel implements
# --------------------------------------------------------------------------------------------------
def _chunk_segment(q, k, v, g, beta, scale, state, chunk):
    """One document of one batch row, all heads: ``q,k [T,H,K]``, ``v [T,H,V]``, ``state [H,K,V]``.

    Per chunk of ``c <= chunk`` tokens, with ``gam`` the in-chunk inclusive cumsum of ``g``:
    ``A_tj = beta_t exp(gam_t - gam_j) k_t.k_j`` (j < t), ``T = (I + A)^-1``,
    ``X = diag(beta) V - diag(beta exp(gam)) K S``, ``Delta = T X``,
    ``O = scale (diag(exp(gam)) Q S + ((Q K^T) o M) Delta)`` with ``M_tj = exp(gam_t - gam_j)`` (j <= t),
    ``S' = exp(gam_c) S + K^T diag(exp(gam_c - gam)) Delta``.
    This is the chunk form of ``gdn_ref.py:17-21`` (FLA's ``kkt_solve`` / ``recompute_w_u`` /
    ``fwd_kernel_h`` / ``fwd_kernel_o`` stages, ``tests/train/test_profiling.py:26-34``), written with
    ``X`` instead of FLA's ``W``/``U`` so that ``K S`` is the only product with the state before the solve.
    """
    t = q.shape[0]
    outs = []
    for c0 in range(0, t, chunk):
        qc, kc, vc = q[c0 : c0 + chunk], k[c0 : c0 + chunk], v[c0 : c0 + chunk]
        gc, bc = g[c0 : c0 + chunk], beta[c0 : c0 + chunk]
        c = qc.shape[0]
        gam = torch.cumsum(gc, 0)  # [c,H]
        idx = torch.arange(c)
        strict = idx[:, None] > idx[None, :]
        causal = idx[:, None] >= idx[None, :]
        diff = gam[:, None, :] - gam[None, :, :]  # [t,j,H]
        decay = torch.where(causal[..., None], diff, torch.full_like(diff, -float("inf"))).exp()
        kk = torch.einsum("thk,jhk->tjh", kc, kc)
        a = torch.where(strict[..., None], bc[:, None, :] * decay * kk, torch.zeros_like(kk))
        eye = torch.eye(c, dtype=q.dtype)
        tmat = torch.linalg.solve_triangular(
            (eye[..., None] + a).permute(2, 0, 1), eye.expand(q.shape[1], c, c), upper=False, unitriangular=True
        )  # [H,c,c]
        ks = torch.einsum("thk,hkv->thv", kc, state)
        x = bc[..., None] * vc - (bc * gam.exp())[..., None] * ks
        delta = torch.einsum("htj,jhv->thv", tmat, x)
        qs = torch.einsum("thk,hkv->thv", qc, state)
        p = torch.where(causal[..., None], torch.einsum("thk,jhk->tjh", qc, kc) * decay, torch.zeros_like(kk))
        outs.append(scale * (gam.exp()[..., None] * qs + torch.einsum("tjh,jhv->thv", p, delta)))
        last = gam[-1]  # [H]
        dt = (last[None, :] - gam).exp()[..., None] * delta
        state = last.exp()[:, None, None] * state + torch.einsum("thk,thv->hkv", kc, dt)
    if outs:
        return torch.cat(outs, 0), state
    return q.new_zeros(0, q.shape[1], v.shape[-1]), state


def chunk_gated_delta_rule_ref(
    q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False, cu_seqlens=None, chunk_size=64
):
    """Chunked gated delta rule in fp64 (same interface as ``recurrent_gated_delta_rule``).

    Chunks restart at every document boundary, as FLA's varlen chunk indices do
    (``sore/model/gdn.py:31-51``: ``n_chunks = sum(ceil(L_i / 64))``).
    """
    b, t, _, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    if scale is None:
        scale = kd**-0.5
    out_dtype = v.dtype
    q, k = gva_expand(q, hv), gva_expand(k, hv)
    q, k, v, g, beta = (x.double() for x in (q, k, v, g, beta))
    if cu_seqlens is None:
        segs = [(bi, 0, t, bi) for bi in range(b)]
    else:
        bounds = _check_cu(cu_seqlens, b, t)
        segs = [(0, a, e, n) for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:]))]
    o = torch.zeros(b, t, hv, vd, dtype=torch.float64)
    finals = []
    for bi, a, e, n in segs:
        s0 = torch.zeros(hv, kd, vd, dtype=torch.float64) if initial_state is None else initial_state[n].double()
        oo, s = _chunk_segment(q[bi, a:e], k[bi, a:e], v[bi, a:e], g[bi, a:e], beta[bi, a:e], scale, s0, chunk_size)
        o[bi, a:e] = oo
        finals.append(s)
    return o.to(out_dtype), (torch.stack(finals) if output_final_state else None)


def _chunk_segment_bwd(q, k, v, g, beta, do, scale, state, dstate, chunk):
    """Backward of ``_chunk_segment`` for one document, all heads, fp64.

    ``q,k [T,H,K]``, ``v,do [T,H,V]``, ``g,beta [T,H]``, ``state [H,K,V]`` (the initial state),
    ``dstate [H,K,V]`` (the gradient of the final state). Returns ``(dq, dk, dv, dg, dbeta, dstate0)``.

    A forward sweep keeps the state entering each chunk; a reverse sweep carries ``dS`` (the
    gradient of the state leaving the chunk). Per chunk, with the forward's names
    (``Y = K S``, ``X``, ``Delta``, ``P = (Q K^T) o M``, ``r = exp(gam_c - gam)``):
    ``dDelta = scale P^T dO + r o (K dS')``, ``dX = T^T dDelta``, ``dV = diag(beta) dX``,
    ``dY = -diag(beta exp(gam)) dX``, ``dA = -strict(dX Delta^T)``, and
    ``dS = exp(gam_c) dS' + scale Q^T diag(exp(gam)) dO + K^T dY``. The gate gradient is the
    reverse in-chunk cumsum of ``dgam``. This is the algebra of FLA's ``chunk_gated_delta_rule_bwd``
    stages (``tests/train/test_profiling.py:25,29,31,32,35``); it is pinned against torch autograd
    through the token recurrence.
    """
    t, h = q.shape[0], q.shape[1]
    starts = list(range(0, t, chunk))
    states = []
    s = state
    for c0 in starts:
        states.append(s)
        _, s = _chunk_segment(q[c0 : c0 + chunk], k[c0 : c0 + chunk], v[c0 : c0 + chunk], g[c0 : c0 + chunk],
                              beta[c0 : c0 + chunk], scale, s, chunk)
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dg, db = torch.zeros_like(g), torch.zeros_like(beta)
    ds_next = dstate.clone()
    for ci in range(len(starts) - 1, -1, -1):
        c0 = starts[ci]
        sl = slice(c0, c0 + chunk)
        qc, kc, vc, gc, bc, doc = q[sl], k[sl], v[sl], g[sl], beta[sl], do[sl]
        s = states[ci]
        c = qc.shape[0]
        gam = torch.cumsum(gc, 0)  # [c,H]
        idx = torch.arange(c)
        strict = (idx[:, None] > idx[None, :])[..., None]
        causal = (idx[:, None] >= idx[None, :])[..., None]
        diff = gam[:, None, :] - gam[None, :, :]
        e = torch.where(causal, diff, torch.full_like(diff, -float("inf"))).exp()  # [t,j,H]
        a_vec, r_vec = gam.exp(), (gam[-1][None, :] - gam).exp()  # [c,H]
        ac = gam[-1].exp()  # [H]
        gram = torch.einsum("thk,jhk->tjh", kc, kc)
        amat = torch.where(strict, bc[:, None, :] * e * gram, torch.zeros_like(gram))
        eye = torch.eye(c, dtype=q.dtype)
        tmat = torch.linalg.solve_triangular(
            (eye[..., None] + amat).permute(2, 0, 1), eye.expand(h, c, c), upper=False, unitriangular=True
        )  # [H,t,j]
        y = torch.einsum("thk,hkv->thv", kc, s)
        x = bc[..., None] * vc - (bc * a_vec)[..., None] * y
        delta = torch.einsum("htj,jhv->thv", tmat, x)
        qk = torch.einsum("thk,jhk->tjh", qc, kc)
        p = torch.where(causal, qk * e, torch.zeros_like(qk))
        # reverse
        w1 = torch.einsum("thk,hkv->thv", kc, ds_next)
        ddelta = scale * torch.einsum("tjh,thv->jhv", p, doc) + r_vec[..., None] * w1
        dx = torch.einsum("htj,thv->jhv", tmat, ddelta)
        dv[sl] = bc[..., None] * dx
        dy = -(bc * a_vec)[..., None] * dx
        da = -torch.where(strict, torch.einsum("thv,jhv->tjh", dx, delta), torch.zeros_like(gram))
        dgram = bc[:, None, :] * da * e  # strict by construction
        dp = torch.where(causal, scale * torch.einsum("thv,jhv->tjh", doc, delta), torch.zeros_like(qk))
        dqk = dp * e
        dq_s = scale * a_vec[..., None] * torch.einsum("thv,hkv->thk", doc, s)
        dq[sl] = dq_s + torch.einsum("tjh,jhk->thk", dqk, kc)
        dk_y = torch.einsum("thv,hkv->thk", dy, s)
        dk_r = r_vec[..., None] * torch.einsum("thv,hkv->thk", delta, ds_next)
        dk[sl] = (dk_r + torch.einsum("tjh,thk->jhk", dqk, qc) + torch.einsum("tjh,jhk->thk", dgram, kc)
                  + torch.einsum("tjh,thk->jhk", dgram, kc) + dk_y)
        db[sl] = (da * e * gram).sum(1) + ((vc - a_vec[..., None] * y) * dx).sum(-1)
        pair = dgram * gram + dqk * qk  # [t,j,H]
        dr = r_vec * (w1 * delta).sum(-1)  # r_t dr_t
        dgam = (qc * dq_s).sum(-1) + (kc * dk_y).sum(-1) - dr + pair.sum(1) - pair.sum(0)
        dgam[-1] = dgam[-1] + ac * (s * ds_next).sum((-2, -1)) + dr.sum(0)
        dg[sl] = torch.flip(torch.cumsum(torch.flip(dgam, [0]), 0), [0])
        ds_next = (ac[:, None, None] * ds_next + scale * torch.einsum("thk,thv->hkv", qc, a_vec[..., None] * doc)
                   + torch.einsum("thk,thv->hkv", kc, dy))
    return dq, dk, dv, dg, db, ds_next


def chunk_gated_delta_rule_bwd_ref(
    q, k, v, g, beta, do, scale=None, initial_state=None, dht=None, cu_seqlens=None, chunk_size=64
):
    """Gradients of ``chunk_gated_delta_rule_ref`` in fp64: ``(dq, dk, dv, dg, dbeta, dh0)``.

    ``do [B,T,HV,V]`` is the gradient of ``o``; ``dht [N,HV,K,V]`` (or ``None``) that of the final
    state. ``dq, dk`` come back in the q/k layout ``[B,T,H,K]`` (summed over the value heads that
    share a q/k head, the adjoint of ``gva_expand``); ``dh0 [N,HV,K,V]``. All fp64. This is the
    backward the reference gets from torch autograd through ``sore/model/gdn_ref.py:11-22``, written
    in chunk form.
    """
    b, t, h, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    if scale is None:
        scale = kd**-0.5
    qe, ke = gva_expand(q, hv), gva_expand(k, hv)
    qe, ke, v, g, beta, do = (x.double() for x in (qe, ke, v, g, beta, do))
    if cu_seqlens is None:
        segs = [(bi, 0, t, bi) for bi in range(b)]
    else:
        bounds = _check_cu(cu_seqlens, b, t)
        segs = [(0, a, e, n) for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:]))]
    dq, dk = torch.zeros(b, t, hv, kd, dtype=torch.float64), torch.zeros(b, t, hv, kd, dtype=torch.float64)
    dv = torch.zeros(b, t, hv, vd, dtype=torch.float64)
    dg, db = torch.zeros(b, t, hv, dtype=torch.float64), torch.zeros(b, t, hv, dtype=torch.float64)
    dh0 = torch.zeros(len(segs), hv, kd, vd, dtype=torch.float64)
    for bi, a, e, n in segs:
        s0 = torch.zeros(hv, kd, vd, dtype=torch.float64) if initial_state is None else initial_state[n].double()
        ds = torch.zeros(hv, kd, vd, dtype=torch.float64) if dht is None else dht[n].double()
        r = _chunk_segment_bwd(qe[bi, a:e], ke[bi, a:e], v[bi, a:e], g[bi, a:e], beta[bi, a:e], do[bi, a:e],
                               scale, s0, ds, chunk_size)
        dq[bi, a:e], dk[bi, a:e], dv[bi, a:e], dg[bi, a:e], db[bi, a:e], dh0[n] = r
    rep = hv // h
    dq = dq.view(b, t, h, rep, kd).sum(3)
    dk = dk.view(b, t, h, rep, kd).sum(3)
    return dq, dk, dv, dg, db, dh0


# --------------------------------------------------------------------------------------------------
# prologue: causal depthwise conv + SiLU, L2 norm, gates  (sore/model/conv.py, gdn.py)
# --------------------------------------------------------------------------------------------------
def causal_conv1d_varlen(x: Tensor, weight: Tensor, doc_ids: Tensor | None) -> Tensor:
    """``y_t = sum_j weight[:, K-1-j] x_{t-j}`` with terms from another document masked out.

    Restates ``sore/model/conv.py:6-23``: ``weight[:, K-1]`` multiplies the current token; a term
    from another document is removed with ``masked_fill`` (never multiplied by 0, so a NaN there
    cannot leak). ``x [B,T,C]``, ``weight [C,K]``, ``doc_ids LongTensor[T]`` or ``None``.
    """
    t = x.shape[1]
    kw = weight.shape[1]
    out = x * weight[:, kw - 1]
    for j in range(1, min(kw, t)):
        term = x[:, : t - j] * weight[:, kw - 1 - j]
        if doc_ids is not None:
            same = doc_ids[j:] == doc_ids[: t - j]
            term = term.masked_fill(~same[None, :, None], 0.0)
        out = out + F.pad(term, (0, 0, j, 0))
    return out


def causal_conv1d_silu(x: Tensor, weight: Tensor, cu_seqlens: Tensor | None = None, activation: str | None = "silu"):
    """Conv + SiLU with fp32 math and one rounding to ``x.dtype``.

    This is the ``gdn_fla_conv`` variant (``sore/model/gdn.py:199-207``: FLA reads the fp32 weight
    directly). The torch variant (``gdn.py:208-209``) casts the weight to the activation dtype first;
    the two differ only by bf16 rounding.
    """
    ids = None if cu_seqlens is None else doc_ids_from_cu_seqlens(cu_seqlens, x.shape[1])
    y = causal_conv1d_varlen(x.double(), weight.double(), ids)
    if activation in ("silu", "swish"):
        y = F.silu(y)
    elif activation is not None:
        raise ValueError(f"unsupported activation {activation!r}")
    return y.to(x.dtype)


def conv_state_from_sequence(x: Tensor, width: int, cu_seqlens: Tensor | None = None) -> Tensor:
    """The rolling conv cache after a prefill: the last ``width`` inputs of each sequence.

    ``x [B,T,C]`` -> ``[N,C,width]``; ``[..., width-1]`` is the newest input, positions before the
    start of a sequence are 0. This is the window the decode step shifts (``legacy/cpp/scripts/chat.py:115-139``
    keeps the same newest-last orientation as ``sore/model/conv.py:7``).
    """
    if cu_seqlens is None:
        segs = [(bi, 0, x.shape[1]) for bi in range(x.shape[0])]
    else:
        bounds = [int(v) for v in cu_seqlens.tolist()]
        segs = [(0, a, e) for a, e in zip(bounds[:-1], bounds[1:])]
    out = x.new_zeros(len(segs), x.shape[2], width)
    for n, (bi, a, e) in enumerate(segs):
        tail = x[bi, max(a, e - width) : e].transpose(0, 1)  # [C, m]
        out[n, :, width - tail.shape[1] :] = tail
    return out


def l2norm(x: Tensor, eps: float = 1e-12) -> Tensor:
    """``F.normalize(x, dim=-1)`` semantics (``sore/model/gdn.py:177``) with fp32 math and one rounding."""
    xf = x.float() if x.dtype != torch.float64 else x
    return (xf / xf.norm(dim=-1, keepdim=True).clamp_min(eps)).to(x.dtype)


def gate_and_beta(a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Tensor):
    """``g = -exp(A_log) softplus(a + dt_bias)`` in fp32 and ``beta = sigmoid(b)`` (``sore/model/gdn.py:191-194``).

    ``a,b [B,T,HV]``; ``A_log, dt_bias [HV]``. Here beta is computed in fp32 (the in-kernel
    ``use_beta_sigmoid_in_kernel`` variant of ``gdn.py:157-162``).
    """
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    return g, b.float().sigmoid()


# --------------------------------------------------------------------------------------------------
# epilogue: RMSNorm and gated RMSNorm  (sore/model/layers.py:7-18, gdn.py:180-188)
# --------------------------------------------------------------------------------------------------
def rms_norm(x: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    """``x rsqrt(mean(x^2) + eps) weight`` in fp32, returned in ``x.dtype`` (``sore/model/layers.py:16-18``)."""
    xf = x.float() if x.dtype != torch.float64 else x
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (out * weight.to(xf.dtype)).to(x.dtype)


def rms_norm_gated(x: Tensor, gate: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    """``RMSNorm(x) * silu(gate)`` with fp32 math and one rounding to ``x.dtype``.

    The fused form used by ``sore/model/gdn.py:182-186`` (``rms_norm_gated(..., activation="swish")``).
    The unfused form at ``gdn.py:188`` rounds ``o_norm(o)`` to the activation dtype before the
    product; the two differ by one bf16 rounding.
    """
    cdt = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf, gf = x.to(cdt), gate.to(cdt)
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.to(cdt)
    return (out * F.silu(gf)).to(x.dtype)


# --------------------------------------------------------------------------------------------------
# decode step: conv-cache update + SiLU + L2 norm + one recurrent token
# --------------------------------------------------------------------------------------------------
def decode_step_ref(
    x_qkv: Tensor,
    conv_state: Tensor,
    conv_weight: Tensor,
    g: Tensor,
    beta: Tensor,
    state: Tensor,
    n_qk_heads: int,
    n_v_heads: int,
    head_dim: int,
    scale: float | None = None,
    use_qk_l2norm: bool = True,
):
    """One decode token for every sequence; returns ``(o [B,1,HV,V], new conv_state, new state)``.

    ``x_qkv [B,C]`` is the pre-conv q|k|v projection (``C = 2 H K + HV V``), ``conv_state [B,C,W]``
    (newest input last), ``conv_weight [C,W]`` fp32, ``g,beta [B,HV]`` fp32, ``state [B,HV,K,V]``.
    The conv output equals the last row of ``causal_conv1d_varlen`` over the history
    (``sore/model/conv.py:6-23``, then ``F.silu``, ``gdn.py:209``); q/k are L2-normalised
    (``gdn.py:177``); the state update is one step of ``gdn_ref.py:17-21``.

    Rounding points: the conv + SiLU output is rounded once to ``x_qkv.dtype`` (as the prefill conv
    kernel and FLA's ``causal_conv1d`` do); the L2 norm and the recurrence then run in fp32 with no
    further rounding until ``o``.
    """
    b, c = x_qkv.shape
    window = torch.cat([conv_state[..., 1:].float(), x_qkv.float()[..., None]], dim=-1)  # [B,C,W]
    y = F.silu((window.double() * conv_weight.double()[None]).sum(-1)).to(x_qkv.dtype).float()
    new_conv = window.to(conv_state.dtype)
    qd = n_qk_heads * head_dim
    if c != 2 * qd + n_v_heads * head_dim:
        raise ValueError(f"x_qkv has {c} channels, expected {2 * qd + n_v_heads * head_dim}")
    q = y[:, :qd].view(b, 1, n_qk_heads, head_dim)
    k = y[:, qd : 2 * qd].view(b, 1, n_qk_heads, head_dim)
    v = y[:, 2 * qd :].view(b, 1, n_v_heads, head_dim)
    if use_qk_l2norm:
        q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        k = k / k.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    o, s = recurrent_gated_delta_rule(
        q, k, v, g[:, None].float(), beta[:, None].float(), scale, initial_state=state, output_final_state=True
    )
    return o.to(x_qkv.dtype), new_conv, s
