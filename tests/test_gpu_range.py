"""GPU: outputs past the fp16 range of the chunked forward's matrix-core operands, and the range guard.

The chunk kernel feeds S, X, Delta, T - I and scale * P to the matrix cores as fp16 (largest finite
value 65504). Values past that range are legal bf16 inputs and FLA (bf16 operands, fp32 exponent
range) returns finite outputs for them. The case used here is v of order 1e5 with L2-normalised
q/k: X = beta (V - e^gam K S) passes 65504 while the fp32 recurrence (the oracle and the recurrent
kernel) stays finite. A slice of the kernel that stores an inf or NaN computes its columns again
by the fp32 recurrence before it exits, so the call returns finite outputs that meet the
north-star bars at the input's scale, and leaves the range flag clear.

The flag is set only when that recomputation is non-finite too: non-finite inputs (FLA returns
non-finite outputs for them as well). The guard's modes, exercised with an inf in v:
  warn      the flag is set, the next call warns and clears it, check_chunk_range() reports it;
  raise     the call raises FloatingPointError;
  fallback  the call returns the fp32 recurrent kernel's result (compared with
            fused_recurrent_gated_delta_rule, NaN positions included); with grad it raises, since
            the backward needs the chunk forward.
Ordinary inputs (the unit-scale synthetic ones, the reference's x100 layer inputs in
test_gpu_layer.py) leave the flag clear. The allocation-free entry point sets the same flag.
"""
import pytest
import torch

import sorernn_amd
from oracle import recurrent_gated_delta_rule
from sorernn_amd import _lib, chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
from sorernn_amd.synthetic import gdn_inputs
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
BIG = 1.0e5


@pytest.fixture(autouse=True)
def _restore_mode():
    yield
    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()


def _inputs(scale_v=1.0, seed=70, inf_at=None):
    inp = gdn_inputs(1, 130, 2, 128, dtype=torch.bfloat16, seed=seed, h0=True)
    inp.v = (inp.v.float() * scale_v).to(torch.bfloat16)
    if inf_at is not None:
        inp.v[0, inf_at, 0, 0] = float("inf")
    return inp


def _nonfinite(seed=70):
    """An inf in v at token 100 (head 0, column 0): every later output of that head is non-finite."""
    return _inputs(seed=seed, inf_at=100)


def _run(inp, **kw):
    d = inp.to(DEV)
    return chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                  output_final_state=True, **kw)


def test_ordinary_inputs_leave_the_flag_clear():
    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    o, st = _run(_inputs())
    assert not sorernn_amd.check_chunk_range()
    assert torch.isfinite(o).all() and torch.isfinite(st).all()


@pytest.mark.parametrize("varlen", [False, True], ids=["fixed", "varlen"])
def test_fp16_overflow_is_recomputed_in_fp32(varlen):
    """v x 1e5: the slices that overflowed fp16 recompute their columns in fp32 inside the kernel; the
    outputs are finite, meet the bars at the input's scale, and the flag stays clear."""
    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    print(f"v x {BIG:g}: chunk kernel, varlen={varlen}", flush=True)
    if varlen:
        cu = torch.tensor([0, 40, 41, 300], dtype=torch.long)
        inp = gdn_inputs(1, 300, 2, 128, HV=4, dtype=torch.bfloat16, seed=72, h0=True, cu_seqlens=cu)
        inp.v = (inp.v.float() * BIG).to(torch.bfloat16)
    else:
        inp = _inputs(BIG)
    d = inp.to(DEV)
    o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                   output_final_state=True, cu_seqlens=d.cu_seqlens, cu_seqlens_cpu=inp.cu_seqlens)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(st).all()
    cu_l = None if inp.cu_seqlens is None else inp.cu_seqlens.long()
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True,
                                               cu_seqlens=cu_l)
    # the north-star bars at the input's scale: outputs divided by BIG, states by relative L2
    assert_output_close((o.float().cpu() / BIG).to(torch.bfloat16), o_ref.float() / BIG, what="o / 1e5")
    assert_state_close(st.cpu(), st_ref, what="final state")
    assert not sorernn_amd.check_chunk_range()


def test_overflow_with_grad_gives_finite_forward():
    """The training forward (it saves the chunk states for the backward) recovers the same way."""
    inp = _inputs(BIG)
    d = inp.to(DEV)
    q = d.q.clone().requires_grad_(True)
    o, st = chunk_gated_delta_rule(q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                   output_final_state=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(st).all()
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    assert_output_close((o.detach().float().cpu() / BIG).to(torch.bfloat16), o_ref.float() / BIG, what="o / 1e5")


def test_nonfinite_inputs_set_the_flag_and_the_next_call_warns():
    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    o, st = _run(_nonfinite())
    torch.cuda.synchronize()
    assert not torch.isfinite(o).all(), "premise: an inf input gives non-finite outputs"
    assert sorernn_amd.check_chunk_range(clear=False)
    with pytest.warns(RuntimeWarning, match="inf or NaN"):
        _run(_inputs())  # an ordinary call reports the earlier one and clears the flag
    assert not sorernn_amd.check_chunk_range()


def test_nonfinite_inputs_raise_in_raise_mode():
    sorernn_amd.set_range_guard("raise")
    with pytest.raises(FloatingPointError, match="fp16 operand"):
        _run(_nonfinite())
    _run(_inputs())  # the flag was cleared: an ordinary call passes


def test_nonfinite_inputs_fall_back_to_the_recurrent_kernel():
    sorernn_amd.set_range_guard("fallback")
    inp = _nonfinite()
    with pytest.warns(RuntimeWarning):
        o, st = _run(inp)
    d = inp.to(DEV)
    o_rec, st_rec = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale,
                                                     initial_state=d.h0, output_final_state=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(o.cpu(), o_rec.cpu(), rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(st.cpu(), st_rec.cpu(), rtol=0, atol=0, equal_nan=True)
    # the finite head (head 1) matches the oracle
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    assert_output_close(o[:, :, 1].cpu(), o_ref[:, :, 1], what="fallback o, finite head")
    assert not sorernn_amd.check_chunk_range()


def test_fallback_with_grad_raises():
    sorernn_amd.set_range_guard("fallback")
    d = _nonfinite().to(DEV)
    q = d.q.clone().requires_grad_(True)
    with pytest.raises(FloatingPointError, match="backward"):
        chunk_gated_delta_rule(q, d.k, d.v, d.g, d.beta, scale=d.scale, initial_state=d.h0)


def test_noalloc_entry_sets_the_same_flag():
    sorernn_amd.set_range_guard("warn")
    _run(_inputs())  # registers the flag word of this device
    sorernn_amd.check_chunk_range()
    inp = _nonfinite(seed=71)
    d = inp.to(DEV)
    b, t, h, kd = d.q.shape
    o = torch.empty_like(d.v)
    fin = torch.empty(b, 2, kd, kd, device=DEV)
    _lib.call("gdn_chunk_fwd_noalloc", d.q.data_ptr(), d.k.data_ptr(), d.v.data_ptr(), d.g.data_ptr(),
              d.beta.data_ptr(), d.h0.data_ptr(), o.data_ptr(), fin.data_ptr(), None, b, t, h, 2, kd, kd, b,
              _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32, inp.scale, 0, None, None, _lib.stream_of(o))
    assert sorernn_amd.check_chunk_range()


def test_off_mode_unregisters_the_flag():
    sorernn_amd.set_range_guard("off")
    _run(_nonfinite())
    assert not sorernn_amd.check_chunk_range()
    sorernn_amd.set_range_guard("warn")
    _run(_inputs())
    assert not sorernn_amd.check_chunk_range()


def test_set_range_flag_rejects_pageable_memory():
    import ctypes

    word = ctypes.c_uint(0)
    lib = _lib.load()
    assert lib.gdn_set_range_flag(torch.cuda.current_device(), ctypes.addressof(word)) == _lib.GDN_ERR_INVALID
    assert b"pinned host memory" in lib.gdn_last_error()
    _run(_inputs())  # the failed query left no error behind for the next launch
