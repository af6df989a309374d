"""``torch.library`` registration of the chunked gated delta rule (forward and backward).

``chunk_gated_delta_rule`` with bf16 q/k/v runs through the two custom ops defined here:

- ``sorernn::chunk_gated_delta_rule_fwd`` -> ``(o, final_state, chunk_states, workspace)``: the
  forward (``gdn_chunk_fwd``), or with ``save_states`` the training forward
  (``gdn_chunk_fwd_train``), whose bf16 per-chunk states and workspace the backward reads;
- ``sorernn::chunk_gated_delta_rule_bwd`` -> ``(dq, dk, dv, dg, dbeta, dh0, dA_log, ddt_bias)``
  (``gdn_chunk_bwd``), tied to the forward with ``register_autograd``.

Both have fake (shape-only) implementations, so ``torch.compile`` traces a block through the op
without a graph break and ``make_fx`` records it as one node. The reference's per-Block
``torch.compile`` breaks its graph at FLA's autograd function (``RUNBOOK_4090.md:203-208``,
``sore/train/trainer.py:99-103``). Absent optional outputs are empty tensors; the public wrapper
in ``ops.py`` turns them back into ``None``.
"""
import os
from typing import Optional

import torch
from torch import Tensor

from sorernn_amd import _lib

C = 64  # chunk length


def _align256(x):
    return (x + 255) // 256 * 256


def fwd_workspace_bytes(b, t, hv, n, varlen: bool):
    """``gdn_chunk_workspace_size`` in Python arithmetic (symbolic sizes allowed under tracing): the
    two-kernel prefill's T - I rows (the larger of those and the cooperative prefill's package ring,
    47,360 bytes per slot, min(8, ceil(T / 64)) slots per chain, with its sync words, 72 per chain + 1,
    while SORERNN_PREFILL=coop selects that route), then the varlen index arrays."""
    nb = _align256(b * t * hv * C * 2)
    if os.environ.get("SORERNN_PREFILL") == "coop":
        slots = torch.sym_min(8, torch.sym_max(1, (t + C - 1) // C))
        coop = _align256(n * hv * slots * 47360) + _align256((n * hv * 72 + 1) * 4)
        nb = torch.sym_max(nb, coop)
    if varlen:
        nb = nb + _align256((n + 1) * 4) + _align256(n * 4)
    return nb


def states_bytes(b, t, hv, kd, vd, n, varlen: bool):
    """``gdn_chunk_states_size``: one bf16 K x V state per chunk and value head."""
    chunks = ((t + C - 1) // C + n) if varlen else b * ((t + C - 1) // C)
    return chunks * hv * kd * vd * 2


def bwd_workspace_bytes(b, t, hv, kd, vd, n, varlen: bool):
    """``gdn_chunk_bwd_workspace_size``."""
    tok = b * t
    chunks = ((t + C - 1) // C + n) if varlen else b * ((t + C - 1) // C)
    return (_align256(tok * hv * C * 2) + _align256(chunks * hv * vd * C * 2) + _align256(chunks * hv * kd * vd * 2)
            + _align256(chunks * hv * 2 * 4))


def chunk_fwd_impl(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, initial_state: Optional[Tensor],
              A_log: Optional[Tensor], dt_bias: Optional[Tensor], cu_seqlens: Optional[Tensor], scale: float,
              flags: int, num_seqs: int, output_final_state: bool,
              save_states: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    b, t, h, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    n = num_seqs
    qc, kc, vc, gc, bc = (x.contiguous() for x in (q, k, v, g, beta))
    h0 = None if initial_state is None else initial_state.float().contiguous()
    al = None if A_log is None else A_log.float().contiguous()
    dtb = None if dt_bias is None else dt_bias.float().contiguous()
    cu = None if cu_seqlens is None else cu_seqlens.contiguous()
    varlen = cu is not None
    dev = q.device
    o = torch.empty(b, t, hv, vd, device=dev, dtype=q.dtype)
    final = torch.empty((n, hv, kd, vd) if output_final_state else (0,), device=dev, dtype=torch.float32)
    ws = torch.empty(max(fwd_workspace_bytes(b, t, hv, n, varlen), 1), device=dev, dtype=torch.uint8)
    states = torch.empty(states_bytes(b, t, hv, kd, vd, n, varlen) if save_states else 0, device=dev,
                         dtype=torch.uint8)
    fin = final if output_final_state else None
    if t > 0:
        args = [_lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(gc), _lib.ptr(bc), _lib.ptr(h0), _lib.ptr(o),
                _lib.ptr(fin), _lib.ptr(cu), b, t, h, hv, kd, vd, n, _lib.dtype_code(qc.dtype),
                _lib.dtype_code(gc.dtype), _lib.dtype_code(bc.dtype), scale, flags, _lib.ptr(al), _lib.ptr(dtb)]
        if save_states:
            _lib.call("gdn_chunk_fwd_train", *args, _lib.ptr(states), _lib.ptr(ws), ws.numel(), _lib.stream_of(qc))
        else:
            _lib.call("gdn_chunk_fwd", *args, _lib.ptr(ws), ws.numel(), _lib.stream_of(qc))
    elif fin is not None:
        fin.copy_(h0 if h0 is not None else torch.zeros_like(fin))
    return o, final, states, ws


# The registered op; ``chunk_fwd_impl`` is its implementation, which the eager inference path of
# ``ops.py`` calls directly (no dispatcher round trip when nothing traces, records or differentiates).
chunk_fwd = torch.library.custom_op("sorernn::chunk_gated_delta_rule_fwd", mutates_args=())(chunk_fwd_impl)


@chunk_fwd.register_fake
def _chunk_fwd_fake(q, k, v, g, beta, initial_state, A_log, dt_bias, cu_seqlens, scale, flags, num_seqs,
                    output_final_state, save_states):
    b, t, _, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    varlen = cu_seqlens is not None
    o = q.new_empty(b, t, hv, vd)
    final = q.new_empty((num_seqs, hv, kd, vd) if output_final_state else (0,), dtype=torch.float32)
    states = q.new_empty(states_bytes(b, t, hv, kd, vd, num_seqs, varlen) if save_states else 0, dtype=torch.uint8)
    ws = q.new_empty(max(fwd_workspace_bytes(b, t, hv, num_seqs, varlen), 1), dtype=torch.uint8)
    return o, final, states, ws


@torch.library.custom_op("sorernn::chunk_gated_delta_rule_bwd", mutates_args=())
def chunk_bwd(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, d_o: Tensor, d_final_state: Optional[Tensor],
              chunk_states: Tensor, fwd_workspace: Tensor, A_log: Optional[Tensor], dt_bias: Optional[Tensor],
              cu_seqlens: Optional[Tensor], scale: float, flags: int, num_seqs: int,
              initial_state_grad: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    b, t, h, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    n = num_seqs
    qc, kc, vc, gc, bc = (x.contiguous() for x in (q, k, v, g, beta))
    do = d_o.to(qc.dtype).contiguous()
    dht = None if d_final_state is None else d_final_state.float().contiguous()
    al = None if A_log is None else A_log.float().contiguous()
    dtb = None if dt_bias is None else dt_bias.float().contiguous()
    cu = None if cu_seqlens is None else cu_seqlens.contiguous()
    dev = q.device
    dq, dk, dv = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
    dg, db = torch.empty_like(gc), torch.empty_like(bc)
    dh0 = torch.empty((n, hv, kd, vd) if initial_state_grad else (0,), device=dev, dtype=torch.float32)
    gate = bool(flags & _lib.FLAG_GATE_IN_KERNEL)
    dal = torch.empty(hv if gate else 0, device=dev, dtype=torch.float32)
    ddt = torch.empty(hv if gate else 0, device=dev, dtype=torch.float32)
    if t > 0:
        bws = torch.empty(max(bwd_workspace_bytes(b, t, hv, kd, vd, n, cu is not None), 1), device=dev,
                          dtype=torch.uint8)
        _lib.call("gdn_chunk_bwd", _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(gc), _lib.ptr(bc), _lib.ptr(do),
                  _lib.ptr(dht), _lib.ptr(chunk_states), _lib.ptr(fwd_workspace), _lib.ptr(cu), b, t, h, hv, kd, vd, n,
                  _lib.dtype_code(qc.dtype), _lib.dtype_code(gc.dtype), _lib.dtype_code(bc.dtype), scale, flags,
                  _lib.ptr(al), _lib.ptr(dtb), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(db),
                  _lib.ptr(dh0 if initial_state_grad else None), _lib.ptr(dal if gate else None),
                  _lib.ptr(ddt if gate else None), _lib.ptr(bws), bws.numel(), _lib.stream_of(qc))
    else:
        if initial_state_grad:
            dh0.copy_(dht if dht is not None else torch.zeros_like(dh0))
        dal.zero_()
        ddt.zero_()
    return dq, dk, dv, dg, db, dh0, dal, ddt


@chunk_bwd.register_fake
def _chunk_bwd_fake(q, k, v, g, beta, d_o, d_final_state, chunk_states, fwd_workspace, A_log, dt_bias, cu_seqlens,
                    scale, flags, num_seqs, initial_state_grad):
    _, _, _, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    gate = bool(flags & _lib.FLAG_GATE_IN_KERNEL)
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(g), torch.empty_like(beta),
            q.new_empty((num_seqs, hv, kd, vd) if initial_state_grad else (0,), **f32),
            q.new_empty(hv if gate else 0, **f32), q.new_empty(hv if gate else 0, **f32))


def _setup_context(ctx, inputs, output):
    q, k, v, g, beta, initial_state, A_log, dt_bias, cu_seqlens, scale, flags, num_seqs, _, save_states = inputs
    _, _, states, ws = output
    if not save_states:
        raise RuntimeError("sorernn::chunk_gated_delta_rule_fwd: a backward needs save_states=True")
    ctx.save_for_backward(q, k, v, g, beta, A_log, dt_bias, cu_seqlens, states, ws)
    ctx.meta = (scale, flags, num_seqs)
    ctx.h0_dtype = None if initial_state is None else initial_state.dtype
    ctx.param_dtypes = (None if A_log is None else A_log.dtype, None if dt_bias is None else dt_bias.dtype)
    ctx.set_materialize_grads(False)


def _backward(ctx, d_o, d_final, _d_states, _d_ws):
    q, k, v, g, beta, A_log, dt_bias, cu_seqlens, states, ws = ctx.saved_tensors
    scale, flags, num_seqs = ctx.meta
    if d_o is None:
        d_o = torch.zeros(q.shape[0], q.shape[1], v.shape[2], v.shape[3], device=q.device, dtype=q.dtype)
    if d_final is not None and d_final.numel() == 0:
        d_final = None
    want_h0 = ctx.h0_dtype is not None and ctx.needs_input_grad[5]
    dq, dk, dv, dg, db, dh0, dal, ddt = chunk_bwd(q, k, v, g, beta, d_o, d_final, states, ws, A_log, dt_bias,
                                                  cu_seqlens, scale, flags, num_seqs, want_h0)
    gate = bool(flags & _lib.FLAG_GATE_IN_KERNEL)
    return (dq, dk, dv, dg, db, dh0.to(ctx.h0_dtype) if want_h0 else None,
            dal.to(ctx.param_dtypes[0]) if gate else None, ddt.to(ctx.param_dtypes[1]) if gate else None,
            None, None, None, None, None, None)


chunk_fwd.register_autograd(_backward, setup_context=_setup_context)


# ---------------------------------------------------------------------------------------------------
# causal conv1d (+ SiLU): sorernn::causal_conv1d_fwd / _bwd
# ---------------------------------------------------------------------------------------------------
@torch.library.custom_op("sorernn::causal_conv1d_fwd", mutates_args=())
def conv_fwd(x: Tensor, weight: Tensor, bias: Optional[Tensor], initial_state: Optional[Tensor],
             cu_seqlens: Optional[Tensor], activation: int, flags: int, num_seqs: int,
             output_final_state: bool) -> tuple[Tensor, Tensor]:
    b, t, c = x.shape
    w = weight.shape[1]
    xc = x.contiguous()
    init = None if initial_state is None else initial_state.to(x.dtype).contiguous()
    wgt = weight.float().contiguous()
    bs = None if bias is None else bias.float().contiguous()
    cu = None if cu_seqlens is None else cu_seqlens.contiguous()
    y = torch.empty_like(xc)
    fin = torch.empty((num_seqs, c, w) if output_final_state else (0,), device=x.device, dtype=x.dtype)
    _lib.call("gdn_causal_conv1d_fwd", _lib.ptr(xc), _lib.ptr(wgt), _lib.ptr(bs), _lib.ptr(y), _lib.ptr(init),
              _lib.ptr(fin if output_final_state else None), _lib.ptr(cu), b, t, c, w, num_seqs,
              _lib.dtype_code(xc.dtype), activation, flags, _lib.stream_of(xc))
    return y, fin


@conv_fwd.register_fake
def _conv_fwd_fake(x, weight, bias, initial_state, cu_seqlens, activation, flags, num_seqs, output_final_state):
    c, w = x.shape[2], weight.shape[1]
    return torch.empty_like(x), x.new_empty((num_seqs, c, w) if output_final_state else (0,))


@torch.library.custom_op("sorernn::causal_conv1d_bwd", mutates_args=())
def conv_bwd(x: Tensor, weight: Tensor, bias: Optional[Tensor], initial_state: Optional[Tensor],
             cu_seqlens: Optional[Tensor], dy: Tensor, activation: int, flags: int,
             num_seqs: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    b, t, c = x.shape
    w = weight.shape[1]
    xc = x.contiguous()
    init = None if initial_state is None else initial_state.to(x.dtype).contiguous()
    wgt = weight.float().contiguous()
    bs = None if bias is None else bias.float().contiguous()
    cu = None if cu_seqlens is None else cu_seqlens.contiguous()
    dyc = dy.to(x.dtype).contiguous()
    dx = torch.empty_like(xc)
    dw = torch.empty(c, w, device=x.device, dtype=torch.float32)
    db = torch.empty(c if bias is not None else 0, device=x.device, dtype=torch.float32)
    dinit = torch.empty((num_seqs, c, w) if initial_state is not None else (0,), device=x.device, dtype=torch.float32)
    ws = torch.empty(max(int(_lib.load().gdn_causal_conv1d_bwd_workspace_size(b, t, c, w)), 1), device=x.device,
                     dtype=torch.uint8)
    _lib.call("gdn_causal_conv1d_bwd", _lib.ptr(xc), _lib.ptr(wgt), _lib.ptr(bs), _lib.ptr(dyc), _lib.ptr(init),
              _lib.ptr(cu), b, t, c, w, num_seqs, _lib.dtype_code(xc.dtype), activation, flags, _lib.ptr(dx),
              _lib.ptr(dw), _lib.ptr(db if bias is not None else None),
              _lib.ptr(dinit if initial_state is not None else None), _lib.ptr(ws), ws.numel(), _lib.stream_of(xc))
    return dx, dw, db, dinit


@conv_bwd.register_fake
def _conv_bwd_fake(x, weight, bias, initial_state, cu_seqlens, dy, activation, flags, num_seqs):
    c, w = x.shape[2], weight.shape[1]
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(x), x.new_empty((c, w), **f32), x.new_empty(c if bias is not None else 0, **f32),
            x.new_empty((num_seqs, c, w) if initial_state is not None else (0,), **f32))


def _conv_setup(ctx, inputs, output):
    x, weight, bias, initial_state, cu_seqlens, activation, flags, num_seqs, _ = inputs
    ctx.save_for_backward(x, weight, bias, initial_state, cu_seqlens)
    ctx.meta = (activation, flags, num_seqs)
    ctx.set_materialize_grads(False)


def _conv_backward(ctx, dy, dfin):
    if dfin is not None and dfin.numel() > 0:
        raise NotImplementedError("causal_conv1d: no gradient through final_state (the decode cache)")
    x, weight, bias, initial_state, cu_seqlens = ctx.saved_tensors
    activation, flags, num_seqs = ctx.meta
    if dy is None:
        dy = torch.zeros_like(x)
    dx, dw, db, dinit = conv_bwd(x, weight, bias, initial_state, cu_seqlens, dy, activation, flags, num_seqs)
    return (dx, dw.to(weight.dtype), None if bias is None else db.to(bias.dtype),
            None if initial_state is None else dinit.to(initial_state.dtype), None, None, None, None, None)


conv_fwd.register_autograd(_conv_backward, setup_context=_conv_setup)


# ---------------------------------------------------------------------------------------------------
# L2 norm and gated RMSNorm: sorernn::l2norm_fwd / _bwd, sorernn::rms_norm_gated_fwd / _bwd
# ---------------------------------------------------------------------------------------------------
@torch.library.custom_op("sorernn::l2norm_fwd", mutates_args=())
def l2norm_fwd(x: Tensor, eps: float) -> Tensor:
    xc = x.contiguous()
    y = torch.empty_like(xc)
    d = xc.shape[-1]
    _lib.call("gdn_l2norm_fwd", _lib.ptr(xc), _lib.ptr(y), xc.numel() // max(d, 1), d, _lib.dtype_code(xc.dtype), eps,
              _lib.stream_of(xc))
    return y


@l2norm_fwd.register_fake
def _l2norm_fwd_fake(x, eps):
    return torch.empty_like(x)


@torch.library.custom_op("sorernn::l2norm_bwd", mutates_args=())
def l2norm_bwd(x: Tensor, dy: Tensor, eps: float) -> Tensor:
    xc = x.contiguous()
    dyc = dy.to(x.dtype).contiguous()
    dx = torch.empty_like(xc)
    d = xc.shape[-1]
    _lib.call("gdn_l2norm_bwd", _lib.ptr(xc), _lib.ptr(dyc), _lib.ptr(dx), xc.numel() // max(d, 1), d,
              _lib.dtype_code(xc.dtype), eps, _lib.stream_of(xc))
    return dx


@l2norm_bwd.register_fake
def _l2norm_bwd_fake(x, dy, eps):
    return torch.empty_like(x)


def _l2_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.eps = inputs[1]


def _l2_backward(ctx, dy):
    (x,) = ctx.saved_tensors
    return l2norm_bwd(x, dy, ctx.eps), None


l2norm_fwd.register_autograd(_l2_backward, setup_context=_l2_setup)


@torch.library.custom_op("sorernn::rms_norm_gated_fwd", mutates_args=())
def rms_fwd(x: Tensor, gate: Optional[Tensor], weight: Optional[Tensor], bias: Optional[Tensor], eps: float,
            activation: int) -> Tensor:
    xc = x.contiguous()
    gc = None if gate is None else gate.to(xc.dtype).contiguous()
    wc = None if weight is None else weight.float().contiguous()
    bc = None if bias is None else bias.float().contiguous()
    y = torch.empty_like(xc)
    d = xc.shape[-1]
    _lib.call("gdn_rms_norm_gated_fwd", _lib.ptr(xc), _lib.ptr(gc), _lib.ptr(wc), _lib.ptr(bc), _lib.ptr(y),
              xc.numel() // max(d, 1), d, _lib.dtype_code(xc.dtype), eps, activation, _lib.stream_of(xc))
    return y


@rms_fwd.register_fake
def _rms_fwd_fake(x, gate, weight, bias, eps, activation):
    return torch.empty_like(x)


@torch.library.custom_op("sorernn::rms_norm_gated_bwd", mutates_args=())
def rms_bwd(x: Tensor, gate: Optional[Tensor], weight: Optional[Tensor], bias: Optional[Tensor], dy: Tensor,
            eps: float, activation: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    xc = x.contiguous()
    gc = None if gate is None else gate.to(xc.dtype).contiguous()
    wc = None if weight is None else weight.float().contiguous()
    bc = None if bias is None else bias.float().contiguous()
    dyc = dy.to(xc.dtype).contiguous()
    d = xc.shape[-1]
    rows = xc.numel() // max(d, 1)
    dx = torch.empty_like(xc)
    dg = torch.empty_like(xc) if gate is not None else xc.new_empty(0)
    dw = torch.empty(d if weight is not None else 0, device=x.device, dtype=torch.float32)
    db = torch.empty(d if bias is not None else 0, device=x.device, dtype=torch.float32)
    ws = torch.empty(max(int(_lib.load().gdn_rms_norm_gated_bwd_workspace_size(rows, d)), 1), device=x.device,
                     dtype=torch.uint8)
    _lib.call("gdn_rms_norm_gated_bwd", _lib.ptr(xc), _lib.ptr(gc), _lib.ptr(wc), _lib.ptr(bc), _lib.ptr(dyc),
              _lib.ptr(dx), _lib.ptr(dg if gate is not None else None), _lib.ptr(dw if weight is not None else None),
              _lib.ptr(db if bias is not None else None), rows, d, _lib.dtype_code(xc.dtype), eps, activation,
              _lib.ptr(ws), ws.numel(), _lib.stream_of(xc))
    return dx, dg, dw, db


@rms_bwd.register_fake
def _rms_bwd_fake(x, gate, weight, bias, dy, eps, activation):
    d = x.shape[-1]
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(x), torch.empty_like(x) if gate is not None else x.new_empty(0),
            x.new_empty(d if weight is not None else 0, **f32), x.new_empty(d if bias is not None else 0, **f32))


def _rms_setup(ctx, inputs, output):
    x, gate, weight, bias, eps, activation = inputs
    ctx.save_for_backward(x, gate, weight, bias)
    ctx.meta = (eps, activation)


def _rms_backward(ctx, dy):
    x, gate, weight, bias = ctx.saved_tensors
    eps, activation = ctx.meta
    dx, dg, dw, db = rms_bwd(x, gate, weight, bias, dy, eps, activation)
    return (dx, None if gate is None else dg.to(gate.dtype), None if weight is None else dw.to(weight.dtype),
            None if bias is None else db.to(bias.dtype), None, None)


rms_fwd.register_autograd(_rms_backward, setup_context=_rms_setup)
