"""Host-side drop-ins for FLA's GDN operators, launching the gfx950 kernels of ``libgdn.so``.

Each function keeps the signature and argument meaning of the FLA 0.5.2 call it replaces, as used
by soreRNN's ``sore/model/gdn.py`` (the reference's only caller), so the model code changes only
its imports:

- ``chunk_gated_delta_rule``            <- ``fla.ops.gated_delta_rule.chunk_gated_delta_rule`` (gdn.py:151,166-169)
- ``fused_recurrent_gated_delta_rule``  <- ``fla.ops.gated_delta_rule.fused_recurrent_gated_delta_rule``
- ``causal_conv1d``                     <- ``fla.modules.conv.causal_conv1d`` (gdn.py:200-207)
- ``rms_norm_gated``                    <- ``fla.modules.fused_norm_gate.rms_norm_gated`` (gdn.py:182-186)
- ``l2norm``                            <- ``F.normalize(x, dim=-1)`` / FLA ``l2norm`` (gdn.py:177)
- ``gated_delta_decode_step``           (no reference counterpart: the fused decode step)
- ``qkv_causal_conv1d``                 <- the three ``causal_conv1d`` calls + q/k ``l2norm`` of gdn.py:177,199-209, in one pass

Outputs are allocated here from torch's caching allocator; the C ABI never allocates.
``chunk_gated_delta_rule`` (bf16 q/k/v), ``causal_conv1d``, ``l2norm`` and ``rms_norm_gated`` are
differentiable: their backward launches the HIP backward kernels (``gdn_chunk_bwd``,
``gdn_causal_conv1d_bwd``, ``gdn_l2norm_bwd``, ``gdn_rms_norm_gated_bwd``). The chunk op is a
``torch.library`` custom op (``sorernn_amd/library.py``) with a fake implementation and a
registered autograd formula, so ``torch.compile`` traces through it without a graph break; with
grad, its forward also saves the state entering every chunk. The
recurrent/decode operators are forward-only: a call that would need their backward raises
``NotImplementedError`` instead of silently detaching. Contract violations raise ``ValueError`` with the reference's wording
("B == 1", "cu_seqlens"; ``sore/model/gdn_ref.py:42-43,54-55``).
"""
from __future__ import annotations

import warnings

import torch
import torch.nn.functional as F
from torch import Tensor

from sorernn_amd import _lib
from sorernn_amd import library as _library
from sorernn_amd import range_guard as _range

__all__ = [
    "causal_conv1d",
    "chunk_gated_delta_rule",
    "fused_recurrent_gated_delta_rule",
    "gated_delta_decode_step",
    "l2norm",
    "qkv_causal_conv1d",
    "rms_norm_gated",
]


def _no_grad_check(name: str, *tensors) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(
            f"{name}: only the forward pass is implemented on gfx950 (inputs require grad); "
            "run under torch.no_grad() or detach the inputs"
        )


def _check_cuda(name: str, *tensors) -> torch.device:
    first, idx = None, -1
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{name}: every tensor must be on the GPU (got {t.device})")
        d = t.get_device()  # an int: cheaper than building a torch.device per tensor
        if first is None:
            first, idx = t, d
        elif d != idx:
            raise ValueError(f"{name}: tensors on different devices ({first.device} vs {t.device})")
    return None if first is None else first.device


def _cu_info(name: str, cu_seqlens: Tensor | None, cu_seqlens_cpu: Tensor | None, batch: int, t: int):
    """Validate ``cu_seqlens`` and return (number of sequences, flags bits).

    The bounds are checked on ``cu_seqlens_cpu`` when given (no device sync); otherwise the device
    tensor is copied to the host once, as FLA does when it builds its chunk indices.
    """
    if cu_seqlens is None:
        return batch, 0
    if batch != 1:
        raise ValueError(f"{name}: cu_seqlens requires B == 1, got B = {batch}")
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"{name}: cu_seqlens must be 1-D with at least 2 entries")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name}: cu_seqlens must be int32 or int64, got {cu_seqlens.dtype}")
    flags = _lib.FLAG_CU_INT32 if cu_seqlens.dtype == torch.int32 else 0
    if torch.compiler.is_compiling():
        # under torch.compile the values are not read (no host sync, no graph break); the kernels
        # need only N, and cu_seqlens_cpu is checked when the same call runs eagerly
        return cu_seqlens.numel() - 1, flags
    host = cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens.detach().cpu()
    if host.numel() != cu_seqlens.numel():
        raise ValueError(f"{name}: cu_seqlens_cpu has {host.numel()} entries, cu_seqlens {cu_seqlens.numel()}")
    b = host.tolist()
    if b[0] != 0 or b[-1] != t:
        raise ValueError(f"{name}: cu_seqlens must go from 0 to T = {t}, got {b[0]}..{b[-1]}")
    if any(y <= x for x, y in zip(b[:-1], b[1:])):
        raise ValueError(f"{name}: cu_seqlens must be strictly increasing")
    return len(b) - 1, flags


def _delta_rule_args(name, q, k, v, g, beta, scale, initial_state, cu_seqlens, cu_seqlens_cpu,
                     use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias):
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or v.shape[:2] != q.shape[:2]:
        raise ValueError(f"{name}: expected q,k [B,T,H,K] and v [B,T,HV,V], got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    b, t, h, kd = q.shape
    hv, vd = v.shape[2], v.shape[3]
    if hv % h:
        raise ValueError(f"{name}: value heads ({hv}) must be a multiple of q/k heads ({h})")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"{name}: q, k, v must share a dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    for nm, x in (("g", g), ("beta", beta)):
        if tuple(x.shape) != (b, t, hv):
            raise ValueError(f"{name}: {nm} must be [B,T,HV] = {(b, t, hv)}, got {tuple(x.shape)}")
    n, flags = _cu_info(name, cu_seqlens, cu_seqlens_cpu, b, t)
    if initial_state is not None and tuple(initial_state.shape) != (n, hv, kd, vd):
        raise ValueError(f"{name}: initial_state must be [N,HV,K,V] = {(n, hv, kd, vd)}, got {tuple(initial_state.shape)}")
    if use_qk_l2norm_in_kernel:
        flags |= _lib.FLAG_QK_L2NORM
    if use_beta_sigmoid_in_kernel:
        flags |= _lib.FLAG_BETA_SIGMOID
    if use_gate_in_kernel:
        if A_log is None or dt_bias is None:
            raise ValueError(f"{name}: use_gate_in_kernel needs A_log and dt_bias")
        if A_log.numel() != hv or dt_bias.numel() != hv:
            raise ValueError(f"{name}: A_log and dt_bias must have HV = {hv} entries")
        flags |= _lib.FLAG_GATE_IN_KERNEL
        A_log = A_log.detach().float().contiguous()
        dt_bias = dt_bias.detach().float().contiguous()
    else:
        A_log = dt_bias = None
    if scale is None:
        scale = kd**-0.5
    return b, t, h, kd, hv, vd, n, flags, float(scale), A_log, dt_bias


def _plain_eager(x: Tensor) -> bool:
    """True for an ordinary tensor outside torch.compile, FX tracing and any active dispatch mode."""
    return (type(x) is torch.Tensor and not torch.compiler.is_compiling()
            and not torch.fx._symbolic_trace._is_fx_tracing_flag
            and torch.utils._python_dispatch._get_current_dispatch_mode() is None)


_recurrent_noted: set = set()


def _note_recurrent_route(name: str, dtype: torch.dtype) -> None:
    """Warn once per dtype that non-bf16 q/k/v take the token-by-token kernel (no MFMA)."""
    if dtype not in _recurrent_noted:
        _recurrent_noted.add(dtype)
        warnings.warn(f"{name}: {dtype} q/k/v run on the token-by-token fp32 recurrent kernel, not the chunked "
                      "MFMA prefill (bf16 q/k/v only); cast q/k/v to bfloat16 for the chunked path "
                      "(reported once per dtype)", RuntimeWarning, stacklevel=4)


def _gdn_call(entry, name, q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens, cu_seqlens_cpu,
              use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias,
              inplace_final_state=False):
    _check_cuda(name, q, k, v, g, beta, initial_state, cu_seqlens, A_log, dt_bias)
    a_log_in, dt_bias_in = A_log, dt_bias
    b, t, h, kd, hv, vd, n, flags, scale, A_log, dt_bias = _delta_rule_args(
        name, q, k, v, g, beta, scale, initial_state, cu_seqlens, cu_seqlens_cpu,
        use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias)
    if entry == "gdn_chunk_fwd" and q.dtype != torch.bfloat16:
        # The chunk kernels stage bf16 MFMA operands. fp32/fp16 q/k/v keep their precision on the
        # recurrent kernel, which computes the same recurrence token by token in fp32.
        _note_recurrent_route(name, q.dtype)
        entry = "gdn_recurrent_fwd"
    grad_inputs = [q, k, v, g, beta, initial_state] + ([a_log_in, dt_bias_in] if use_gate_in_kernel else [])
    needs_grad = torch.is_grad_enabled() and any(x is not None and x.requires_grad for x in grad_inputs)
    if needs_grad and (entry != "gdn_chunk_fwd" or inplace_final_state):
        raise NotImplementedError(
            f"{name}: the backward exists for chunk_gated_delta_rule with bf16 q/k/v only (inputs "
            "require grad); run under torch.no_grad() or detach the inputs"
        )
    q_raw, k_raw = q, k
    if (entry == "gdn_chunk_fwd" and (flags & _lib.FLAG_QK_L2NORM) and not needs_grad
            and _l2norm_first(q, n, hv, vd, b * t)):
        q, k = (_l2norm_rows(x) for x in (q, k))
        flags &= ~_lib.FLAG_QK_L2NORM
    if entry == "gdn_chunk_fwd":
        # the torch.library op (sorernn::chunk_gated_delta_rule_fwd): traceable by torch.compile, with
        # the backward registered on it; with grad it also keeps the per-chunk states for the backward.
        # Plain eager inference (no grad, no compile or fake tensors, no dispatch mode recording ops)
        # calls the op's implementation directly: the dispatcher round trip costs more host time
        # than the two kernel launches.
        eager = _plain_eager(q)
        op = _library.chunk_fwd if (needs_grad or not eager) else _library.chunk_fwd_impl
        # the fp16 operand range guard (sorernn_amd/range_guard.py) reads its flag in eager calls only
        word = _range.before_call(q.device) if eager else None
        o, final, _, _ = op(q, k, v, g, beta, initial_state, a_log_in if use_gate_in_kernel else None,
                            dt_bias_in if use_gate_in_kernel else None, cu_seqlens, scale, flags, n,
                            bool(output_final_state), needs_grad)
        if _range.call_overflowed(word, q.device):
            if _range.range_guard() == "raise" or needs_grad:
                raise FloatingPointError(
                    f"{name}: the chunked forward stored inf or NaN outputs (non-finite inputs, or an fp16 "
                    "operand of the chunk kernel past 65504 that its fp32 recomputation did not bring back into range)"
                    + ("; no fallback with grad: the backward needs the chunk forward" if needs_grad else ""))
            _range.note_fallback(name)
            return _gdn_call("gdn_recurrent_fwd", name, q_raw, k_raw, v, g, beta, scale, initial_state,
                             output_final_state, cu_seqlens, cu_seqlens_cpu, use_qk_l2norm_in_kernel,
                             use_beta_sigmoid_in_kernel, use_gate_in_kernel, a_log_in, dt_bias_in)
        return o, (final if output_final_state else None)
    q, k, v, g, beta = (x.contiguous() for x in (q, k, v, g, beta))
    h0 = None
    if initial_state is not None:
        h0 = initial_state if (initial_state.dtype == torch.float32 and initial_state.is_contiguous()) else initial_state.float().contiguous()
    if inplace_final_state:
        if initial_state is None or h0.data_ptr() != initial_state.data_ptr():
            raise ValueError(f"{name}: inplace_final_state needs a contiguous fp32 initial_state")
        final = h0
    elif output_final_state:
        final = torch.empty(n, hv, kd, vd, device=q.device, dtype=torch.float32)
    else:
        final = None
    o = torch.empty(b, t, hv, vd, device=q.device, dtype=q.dtype)
    if t > 0 or final is not None:
        cu = cu_seqlens.contiguous() if cu_seqlens is not None else None
        args = [_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), _lib.ptr(h0),
                _lib.ptr(o), _lib.ptr(final), _lib.ptr(cu), b, t, h, hv, kd, vd, n,
                _lib.dtype_code(q.dtype), _lib.dtype_code(g.dtype), _lib.dtype_code(beta.dtype),
                scale, flags, _lib.ptr(A_log), _lib.ptr(dt_bias)]
        if entry == "gdn_chunk_fwd":
            nbytes = chunk_workspace_bytes(b, t, hv, n, cu is not None)
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
            args += [_lib.ptr(ws), nbytes]
        _lib.call(entry, *args, _lib.stream_of(q))
    return o, final


def chunk_workspace_bytes(batch: int, seqlen: int, num_v_heads: int, num_seqs: int, varlen: bool) -> int:
    """Bytes of device workspace ``gdn_chunk_fwd`` needs (the per-chunk ``(I + A)^-1`` rows)."""
    return int(_lib.load().gdn_chunk_workspace_size(batch, seqlen, num_v_heads, num_seqs, int(varlen)))


def chunk_gated_delta_rule(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    scale: float | None = None,
    initial_state: Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_beta_sigmoid_in_kernel: bool = False,
    allow_neg_eigval: bool = False,
    state_v_first: bool = False,
    cu_seqlens: Tensor | None = None,
    cu_seqlens_cpu: Tensor | None = None,
    cp_context=None,
    use_gate_in_kernel: bool = False,
    A_log: Tensor | None = None,
    dt_bias: Tensor | None = None,
):
    """Chunked gated delta rule forward on gfx950 (fused MFMA prefill, 64-token chunks).

    FLA 0.5.2 signature (``docs/superpowers/plans/2026-10-23-sorernn-v2-core.md:141``) plus the
    gate kwargs soreRNN passes (``sore/model/gdn.py:157-162``). ``q,k [B,T,H,K]``, ``v [B,T,HV,V]``,
    ``g,beta [B,T,HV]``; returns ``(o [B,T,HV,V] in v.dtype, final_state [N,HV,K,V] fp32 or None)``.
    With ``cu_seqlens`` (``[N+1]``, needs ``B == 1``) the state and the chunking restart at every
    document. ``cu_seqlens_cpu`` only serves to validate the bounds without a device sync; the
    kernel's grid depends on ``N`` alone.

    Range: the chunk kernel's matrix-core operands for the state, X, Delta, T - I and scale * P are
    fp16 (largest finite value 65504; FLA's bf16 operands reach fp32's range). L2-normalised q/k
    with activation-scale v stay far inside it (|scale * P| <= scale, states of order |v|). A
    workgroup whose operands leave that range (it stored an inf or NaN) computes its columns again
    by the fp32 token-by-token recurrence before the kernel ends, so finite inputs with finite fp32
    results give finite outputs. The kernel flags the call only when that recomputation is
    non-finite as well (non-finite inputs), and ``sorernn_amd.set_range_guard`` selects the
    response: a warning at the next call (default, no synchronisation), ``FloatingPointError``, or a
    recomputation of the call by the fp32 recurrent kernel. ``sorernn_amd.check_chunk_range()``
    reports the flag on demand.
    fp32/fp16 q/k/v run on the recurrent kernel (a warning says so once per dtype).
    """
    if allow_neg_eigval or state_v_first or cp_context is not None:
        raise NotImplementedError("chunk_gated_delta_rule: allow_neg_eigval, state_v_first and cp_context are not supported")
    return _gdn_call("gdn_chunk_fwd", "chunk_gated_delta_rule", q, k, v, g, beta, scale, initial_state,
                     output_final_state, cu_seqlens, cu_seqlens_cpu, use_qk_l2norm_in_kernel,
                     use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias)


def chunk_gated_delta_rule_gated_norm(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor,
    beta: Tensor,
    gate: Tensor,
    norm_weight: Tensor,
    norm_eps: float = 1e-6,
    norm_split: bool = False,
    scale: float | None = None,
    initial_state: Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_beta_sigmoid_in_kernel: bool = False,
    cu_seqlens: Tensor | None = None,
    cu_seqlens_cpu: Tensor | None = None,
    use_gate_in_kernel: bool = False,
    A_log: Tensor | None = None,
    dt_bias: Tensor | None = None,
):
    """``chunk_gated_delta_rule`` with the layer's gated RMSNorm in the same call (inference).

    Returns ``(rms_norm_gated(o, gate, norm_weight, None, "swish", norm_eps), final_state)`` for the
    ``o`` chunk_gated_delta_rule would return: the call at ``sore/model/gdn.py:166-169`` followed by the
    norm at ``gdn.py:182-186``, equal bit for bit to those two calls here. ``norm_split=True`` rounds
    as the reference's unfused route ``o_norm(o) * F.silu(gate)`` (``gdn.py:188``). ``gate`` has
    ``v``'s shape and dtype (bf16); ``norm_weight [V]``. Inputs must not require grad (the backward of
    the norm needs ``o``). When the chains leave CUs free (two per (sequence, head) at least), the
    norm runs in epilogue workgroups of the chunk kernel's own launch, over each O tile as soon as
    it is stored; otherwise the norm kernel follows in place. A call whose outputs are not finite is
    handled by the range guard as in ``chunk_gated_delta_rule``; its fallback recomputes the call as
    chunk_gated_delta_rule + the norm.
    """
    name = "chunk_gated_delta_rule_gated_norm"
    _check_cuda(name, q, k, v, g, beta, initial_state, cu_seqlens, A_log, dt_bias, gate, norm_weight)
    grad_inputs = [q, k, v, g, beta, initial_state, gate, norm_weight, A_log, dt_bias]
    if torch.is_grad_enabled() and any(x is not None and x.requires_grad for x in grad_inputs):
        raise NotImplementedError(f"{name}: inference only (inputs require grad); use chunk_gated_delta_rule and "
                                  "rms_norm_gated for training")
    if q.dtype != torch.bfloat16 or gate.dtype != v.dtype or gate.shape != v.shape:
        raise ValueError(f"{name}: bf16 q/k/v and a gate of v's shape and dtype are required "
                         f"(got q {q.dtype}, v {tuple(v.shape)} {v.dtype}, gate {tuple(gate.shape)} {gate.dtype})")
    a_log_in, dt_bias_in = A_log, dt_bias
    b, t, h, kd, hv, vd, n, flags, scale, A_log, dt_bias = _delta_rule_args(
        name, q, k, v, g, beta, scale, initial_state, cu_seqlens, cu_seqlens_cpu,
        use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias)
    if norm_weight.shape != (vd,):
        raise ValueError(f"{name}: norm_weight must be [{vd}] (got {tuple(norm_weight.shape)})")
    word = _range.before_call(q.device)
    q_raw, k_raw = q, k
    if (flags & _lib.FLAG_QK_L2NORM) and _l2norm_first(q, n, hv, vd, b * t):
        q, k = (_l2norm_rows(x) for x in (q, k))
        flags &= ~_lib.FLAG_QK_L2NORM
    q, k, v, g, beta, gate = (x.contiguous() for x in (q, k, v, g, beta, gate))
    w = norm_weight.float().contiguous()
    h0 = None if initial_state is None else initial_state.float().contiguous()
    final = torch.empty(n, hv, kd, vd, device=q.device, dtype=torch.float32) if output_final_state else None
    o = torch.empty(b, t, hv, vd, device=q.device, dtype=q.dtype)
    if t > 0:
        cu = cu_seqlens.contiguous() if cu_seqlens is not None else None
        nbytes = int(_lib.load().gdn_chunk_gated_norm_workspace_size(b, t, hv, n, vd, int(cu is not None)))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        _lib.call("gdn_chunk_fwd_gated_norm", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
                  _lib.ptr(h0), _lib.ptr(o), _lib.ptr(final), _lib.ptr(cu), b, t, h, hv, kd, vd, n,
                  _lib.dtype_code(q.dtype), _lib.dtype_code(g.dtype), _lib.dtype_code(beta.dtype), scale, flags,
                  _lib.ptr(A_log), _lib.ptr(dt_bias), _lib.ptr(gate), _lib.ptr(w), float(norm_eps),
                  int(bool(norm_split)), _lib.ptr(ws), nbytes, _lib.stream_of(q))
    elif final is not None:
        final.copy_(h0 if h0 is not None else torch.zeros_like(final))
    if _range.call_overflowed(word, q.device):
        if _range.range_guard() == "raise":
            raise FloatingPointError(f"{name}: the fused chunked forward and norm stored inf or NaN outputs (non-finite "
                                     "inputs, or an fp16 operand of the chunk kernel past 65504)")
        _range.note_fallback(name)
        o2, final = chunk_gated_delta_rule(q_raw, k_raw, v, g, beta, scale=scale, initial_state=initial_state,
                                           output_final_state=output_final_state,
                                           use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                           use_beta_sigmoid_in_kernel=use_beta_sigmoid_in_kernel,
                                           cu_seqlens=cu_seqlens, cu_seqlens_cpu=cu_seqlens_cpu,
                                           use_gate_in_kernel=use_gate_in_kernel, A_log=a_log_in, dt_bias=dt_bias_in)
        if norm_split:
            o = rms_norm_gated(o2, None, norm_weight, None, eps=norm_eps) * F.silu(gate)
        else:
            o = rms_norm_gated(o2, gate, norm_weight, None, activation="swish", eps=norm_eps)
    return o, final


def fused_recurrent_gated_delta_rule(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    g: Tensor | None = None,
    beta: Tensor | None = None,
    scale: float | None = None,
    initial_state: Tensor | None = None,
    output_final_state: bool = False,
    inplace_final_state: bool = False,
    cu_seqlens: Tensor | None = None,
    cu_seqlens_cpu: Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    use_beta_sigmoid_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    A_log: Tensor | None = None,
    dt_bias: Tensor | None = None,
):
    """Token-by-token gated delta rule with the state on chip (the decode step at ``T == 1``).

    Same layouts as ``chunk_gated_delta_rule``. ``g=None`` means no decay and ``beta=None`` means
    ``beta = 1`` (FLA's defaults). With ``inplace_final_state=True`` the final state overwrites
    ``initial_state`` (which must be contiguous fp32) and is returned.
    """
    b, t = q.shape[:2]
    hv = v.shape[2]
    if g is None:
        g = torch.zeros(b, t, hv, device=q.device, dtype=torch.float32)
    if beta is None:
        beta = torch.ones(b, t, hv, device=q.device, dtype=torch.float32)
    return _gdn_call("gdn_recurrent_fwd", "fused_recurrent_gated_delta_rule", q, k, v, g, beta, scale, initial_state,
                     output_final_state or inplace_final_state, cu_seqlens, cu_seqlens_cpu, use_qk_l2norm_in_kernel,
                     use_beta_sigmoid_in_kernel, use_gate_in_kernel, A_log, dt_bias,
                     inplace_final_state=inplace_final_state)


def gated_delta_decode_step(
    x_qkv: Tensor,
    conv_state: Tensor,
    conv_weight: Tensor,
    g: Tensor,
    beta: Tensor,
    state: Tensor,
    num_qk_heads: int,
    num_v_heads: int,
    head_dim: int,
    scale: float | None = None,
    use_qk_l2norm_in_kernel: bool = True,
    use_beta_sigmoid_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    A_log: Tensor | None = None,
    dt_bias: Tensor | None = None,
    out: Tensor | None = None,
) -> Tensor:
    """One fused decode token per sequence; updates ``conv_state`` and ``state`` in place.

    ``x_qkv [B, C]`` (or ``[B,1,C]``) is the pre-conv q|k|v projection with
    ``C = 2*num_qk_heads*head_dim + num_v_heads*head_dim``; ``conv_state [B,C,W]`` (newest input
    last); ``conv_weight [C,W]`` fp32; ``g,beta [B,HV]`` (or ``[B,1,HV]``); ``state [B,HV,D,D]``
    fp32. Returns ``o [B,1,HV,D]`` in ``x_qkv.dtype`` (written into ``out`` when given).
    """
    name = "gated_delta_decode_step"
    # This runs once per generated token, so the host path avoids tensor-producing calls when they
    # would be no-ops (reshape / contiguous / detach / float each build a new tensor object) and reads
    # the stream as a raw handle: validation only, then one ctypes call.
    dev = _check_cuda(name, x_qkv, conv_state, conv_weight, g, beta, state, A_log, dt_bias, out)
    _no_grad_check(name, x_qkv, conv_state, conv_weight, g, beta, state)
    b = x_qkv.shape[0]
    x2 = x_qkv if x_qkv.dim() == 2 and x_qkv.is_contiguous() else x_qkv.reshape(b, -1).contiguous()
    c = x2.shape[1]
    h, hv, d = num_qk_heads, num_v_heads, head_dim
    if c != (2 * h + hv) * d:
        raise ValueError(f"{name}: x_qkv has {c} channels, expected {(2 * h + hv) * d}")
    cs = conv_state.shape
    if len(cs) != 3 or cs[0] != b or cs[1] != c or not conv_state.is_contiguous():
        raise ValueError(f"{name}: conv_state must be a contiguous [B,C,W] = [{b},{c},W] tensor")
    w = cs[2]
    if conv_weight.shape != (c, w):
        raise ValueError(f"{name}: conv_weight must be [C,W] = {(c, w)}")
    if state.shape != (b, hv, d, d) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError(f"{name}: state must be a contiguous fp32 [B,HV,D,D] = {(b, hv, d, d)} tensor")
    g2 = g if g.dim() == 2 and g.is_contiguous() else g.reshape(b, -1).contiguous()
    b2 = beta if beta.dim() == 2 and beta.is_contiguous() else beta.reshape(b, -1).contiguous()
    if g2.shape != (b, hv) or b2.shape != (b, hv):
        raise ValueError(f"{name}: g and beta must be [B,HV] = {(b, hv)}")
    flags = 0
    if use_qk_l2norm_in_kernel:
        flags |= _lib.FLAG_QK_L2NORM
    if use_beta_sigmoid_in_kernel:
        flags |= _lib.FLAG_BETA_SIGMOID
    if use_gate_in_kernel:
        if A_log is None or dt_bias is None:
            raise ValueError(f"{name}: use_gate_in_kernel needs A_log and dt_bias")
        flags |= _lib.FLAG_GATE_IN_KERNEL
        A_log, dt_bias = _f32(A_log), _f32(dt_bias)
    else:
        A_log = dt_bias = None
    wgt = _f32(conv_weight)
    if out is None:
        out = torch.empty(b, 1, hv, d, device=dev, dtype=x_qkv.dtype)
    elif out.shape != (b, 1, hv, d) or out.dtype != x_qkv.dtype or not out.is_contiguous():
        raise ValueError(f"{name}: out must be a contiguous [B,1,HV,D] tensor of x_qkv's dtype")
    dc = _lib.dtype_code
    _lib.call("gdn_decode_step", x2.data_ptr(), conv_state.data_ptr(), wgt.data_ptr(), g2.data_ptr(), b2.data_ptr(),
              state.data_ptr(), out.data_ptr(), b, h, hv, d, w, dc(x2.dtype), dc(conv_state.dtype), dc(g2.dtype),
              dc(b2.dtype), float(d**-0.5 if scale is None else scale), flags, _lib.ptr(A_log), _lib.ptr(dt_bias),
              _lib.raw_stream(dev))
    return out


def _f32(t: Tensor) -> Tensor:
    """``t`` as a contiguous fp32 tensor for a kernel that only reads it (no new tensor when it already is one)."""
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.detach().float().contiguous()


def causal_conv1d(
    x: Tensor,
    weight: Tensor | None = None,
    bias: Tensor | None = None,
    residual: Tensor | None = None,
    initial_state: Tensor | None = None,
    output_final_state: bool = False,
    activation: str | None = None,
    cu_seqlens: Tensor | None = None,
    cu_seqlens_cpu: Tensor | None = None,
):
    """Depthwise causal conv1d (+ SiLU) with per-document reset; returns ``(y, final_state | None)``.

    ``x [B,T,C]``, ``weight [C,W]`` (``weight[:, W-1]`` multiplies the current token, as
    ``sore/model/conv.py:7``), ``bias [C]``. ``initial_state``/``final_state`` are conv caches
    ``[N,C,W]`` (newest input last). ``activation`` is None, "silu" or "swish".
    """
    name = "causal_conv1d"
    if weight is None:
        raise ValueError(f"{name}: weight is required")
    if residual is not None:
        raise NotImplementedError(f"{name}: residual is not supported")
    _check_cuda(name, x, weight, bias, initial_state, cu_seqlens)
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[2]:
        raise ValueError(f"{name}: expected x [B,T,C] and weight [C,W], got {tuple(x.shape)}, {tuple(weight.shape)}")
    b, t, c = x.shape
    w = weight.shape[1]
    n, flags = _cu_info(name, cu_seqlens, cu_seqlens_cpu, b, t)
    if activation in ("silu", "swish"):
        act = _lib.ACT_SILU
    elif activation is None:
        act = _lib.ACT_NONE
    else:
        raise NotImplementedError(f"{name}: activation {activation!r} is not supported")
    if initial_state is not None and tuple(initial_state.shape) != (n, c, w):
        raise ValueError(f"{name}: initial_state must be [N,C,W] = {(n, c, w)}")
    cu = cu_seqlens.contiguous() if cu_seqlens is not None else None
    y, fin = _library.conv_fwd(x, weight, bias, initial_state, cu, act, flags, n, bool(output_final_state))
    return y, (fin if output_final_state else None)


def qkv_causal_conv1d(x: Tensor, weight: Tensor, qk_dim: int, v_dim: int, head_dim: int, activation: str | None = "silu",
                      l2norm: bool = True, cu_seqlens: Tensor | None = None, cu_seqlens_cpu: Tensor | None = None,
                      round_before_activation: bool = False):
    """The GDN layer's q/k/v prologue in one launch (inference): conv + SiLU (+ per-head L2 norm of q, k).

    ``x [B, T, >= 2*qk_dim + v_dim]`` holds the q | k | v projection outputs (its rows may be wider,
    e.g. one fused projection GEMM's output); ``weight [2*qk_dim + v_dim, W=4]`` stacks the three
    conv weights. Returns contiguous ``q, k [B, T, qk_dim]`` and ``v [B, T, v_dim]``, equal to three
    ``causal_conv1d(..., activation)`` calls followed by ``l2norm`` of every q/k head
    (``sore/model/gdn.py:177,199-209``). With ``round_before_activation`` the conv output is rounded
    to ``x.dtype`` before the SiLU, the rounding point of the reference's unfused route
    (``causal_conv1d_varlen`` then ``F.silu``, ``gdn.py:208-209``). Forward only.
    """
    name = "qkv_causal_conv1d"
    _no_grad_check(name, x, weight)
    _check_cuda(name, x, weight, cu_seqlens)
    if x.dim() != 3 or x.stride(2) != 1 or x.shape[2] < 2 * qk_dim + v_dim:
        raise ValueError(f"{name}: x must be [B, T, >= {2 * qk_dim + v_dim}] with a contiguous last axis")
    b, t = x.shape[:2]
    if t > 1 and b > 1 and x.stride(0) != t * x.stride(1):
        raise ValueError(f"{name}: x rows must be evenly strided")
    if tuple(weight.shape) != (2 * qk_dim + v_dim, 4):
        raise ValueError(f"{name}: weight must be [{2 * qk_dim + v_dim}, 4], got {tuple(weight.shape)}")
    if activation in ("silu", "swish"):
        act = _lib.ACT_SILU_ROUNDED if round_before_activation else _lib.ACT_SILU
    elif activation is None:
        act = _lib.ACT_NONE
    else:
        raise NotImplementedError(f"{name}: activation {activation!r} is not supported")
    n, flags = _cu_info(name, cu_seqlens, cu_seqlens_cpu, b, t)
    if l2norm:
        flags |= _lib.FLAG_QK_L2NORM
    stride = x.stride(1) if t > 1 else (x.stride(0) if b > 1 else x.shape[2])
    w = weight.detach().float().contiguous()
    q = torch.empty(b, t, qk_dim, device=x.device, dtype=x.dtype)
    k = torch.empty_like(q)
    v = torch.empty(b, t, v_dim, device=x.device, dtype=x.dtype)
    cu = cu_seqlens.contiguous() if cu_seqlens is not None else None
    _lib.call("gdn_qkv_conv_fwd", x.data_ptr(), stride, w.data_ptr(), None, q.data_ptr(), k.data_ptr(), v.data_ptr(),
              _lib.ptr(cu), b, t, qk_dim, v_dim, head_dim, n, _lib.dtype_code(x.dtype), act, flags, _lib.stream_of(x))
    return q, k, v


_cu_count: dict = {}


def _l2norm_first(q: Tensor, n: int, hv: int, vd: int, tokens: int) -> bool:
    """Whether an inference call with use_qk_l2norm_in_kernel normalises q and k by the row kernel
    before the chunk kernels (which then run without the flag) instead of inside them.

    Inside, each of a chain's V/32 state-kernel workgroups normalises the chain's q/k rows on the
    helper waves that set the step time, ~0.9 us more per chunk step. The row kernel instead costs a
    pass over q and k (read and write) on the whole chip. That pays when the state kernel leaves
    half the CUs or more idle and its chains are long. Measured per call (HIP events): B=2, T=8192,
    16 heads of 128 (32 chains, 128 workgroups): 243 us against 310 us; B=4, T=4096 (256
    workgroups): 180 us against 170 us, so the flag stays in the kernels there."""
    dev = q.get_device()
    cus = _cu_count.get(dev)
    if cus is None:
        cus = _cu_count[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
    return 2 * n * hv * max(1, vd // 32) <= cus and tokens >= 2048 * n


def _l2norm_rows(x: Tensor, eps: float = 1e-12) -> Tensor:
    """``l2norm`` without grad: plain eager calls go to the kernel directly (no dispatcher round trip)."""
    if not _plain_eager(x):
        return _library.l2norm_fwd(x, float(eps))
    xc = x.contiguous()
    y = torch.empty_like(xc)
    d = xc.shape[-1]
    if xc.numel():
        _lib.call("gdn_l2norm_fwd", _lib.ptr(xc), _lib.ptr(y), xc.numel() // d, d, _lib.dtype_code(xc.dtype), float(eps),
                  _lib.stream_of(xc))
    return y


def l2norm(x: Tensor, eps: float = 1e-12) -> Tensor:
    """``x / max(||x||_2, eps)`` over the last axis (``F.normalize`` semantics, fp32 math, one rounding)."""
    _check_cuda("l2norm", x)
    return _library.l2norm_fwd(x, float(eps))


def rms_norm_gated(
    x: Tensor,
    g: Tensor | None,
    weight: Tensor | None,
    bias: Tensor | None = None,
    activation: str = "swish",
    residual: Tensor | None = None,
    prenorm: bool = False,
    residual_in_fp32: bool = False,
    eps: float = 1e-6,
) -> Tensor:
    """``x * rsqrt(mean(x^2) + eps) * weight (+ bias) * act(g)`` per row, fp32 math, one rounding.

    ``activation`` is "swish"/"silu" (``sore/model/gdn.py:186``) or None (gate used as is).
    """
    name = "rms_norm_gated"
    if residual is not None or prenorm:
        raise NotImplementedError(f"{name}: residual/prenorm are not supported")
    if activation in ("swish", "silu"):
        act = _lib.ACT_SILU
    elif activation is None:
        act = _lib.ACT_NONE
    else:
        raise NotImplementedError(f"{name}: activation {activation!r} is not supported")
    _check_cuda(name, x, g, weight, bias)
    if g is not None and g.shape != x.shape:
        raise ValueError(f"{name}: gate shape {tuple(g.shape)} != x shape {tuple(x.shape)}")
    d = x.shape[-1]
    if (weight is not None and weight.numel() != d) or (bias is not None and bias.numel() != d):
        raise ValueError(f"{name}: weight/bias must have {d} entries")
    return _library.rms_fwd(x, g, weight, bias, float(eps), act)
