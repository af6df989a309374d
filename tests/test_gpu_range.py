"""GPU: the range guard of the chunked forward's fp16 matrix-core operands.

The chunk kernel feeds S, X, Delta, T - I and scale * P to the matrix cores as fp16 (largest finite
value 65504). Values past that range are legal bf16 inputs and FLA (bf16 operands, fp32 exponent
range) returns finite outputs for them. The case used here is v of order 1e5 with L2-normalised
q/k. Then X = beta (V - e^gam K S) passes 65504, while the fp32 recurrence (the oracle and the
recurrent kernel) stays finite, so the chunk kernel must report it. The guard's modes:
  warn      the flag is set, the next call warns and clears it, check_chunk_range() reports it;
  raise     the call raises FloatingPointError;
  fallback  the call returns the fp32 recurrent kernel's result (checked bitwise against
            fused_recurrent_gated_delta_rule and against the oracle at the input's scale);
            with grad it raises, since the backward needs the chunk forward.
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


def _inputs(scale_v=1.0, seed=70):
    inp = gdn_inputs(1, 130, 2, 128, dtype=torch.bfloat16, seed=seed, h0=True)
    inp.v = (inp.v.float() * scale_v).to(torch.bfloat16)
    return inp


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


def test_overflow_sets_the_flag_and_the_next_call_warns():
    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    print(f"v x {BIG:g}: chunk kernel, warn mode", flush=True)
    o, st = _run(_inputs(BIG))
    torch.cuda.synchronize()
    assert not (torch.isfinite(o).all() and torch.isfinite(st).all()), "premise: the fp16 operands overflow"
    assert sorernn_amd.check_chunk_range(clear=False)
    with pytest.warns(RuntimeWarning, match="inf or NaN"):
        _run(_inputs())  # an ordinary call reports the earlier one and clears the flag
    assert not sorernn_amd.check_chunk_range()


def test_overflow_raises_in_raise_mode():
    sorernn_amd.set_range_guard("raise")
    with pytest.raises(FloatingPointError, match="fp16 operand"):
        _run(_inputs(BIG))
    _run(_inputs())  # the flag was cleared: an ordinary call passes


def test_overflow_falls_back_to_the_recurrent_kernel():
    sorernn_amd.set_range_guard("fallback")
    inp = _inputs(BIG)
    with pytest.warns(RuntimeWarning):
        o, st = _run(inp)
    d = inp.to(DEV)
    o_rec, st_rec = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale,
                                                     initial_state=d.h0, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(o.cpu(), o_rec.cpu()) and torch.equal(st.cpu(), st_rec.cpu())
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    # the north-star bars at the input's scale: outputs divided by BIG, states by relative L2
    assert_output_close((o.float().cpu() / BIG).to(torch.bfloat16), o_ref.float() / BIG, what="fallback o / 1e5")
    assert_state_close(st.cpu(), st_ref, what="fallback final state")
    assert not sorernn_amd.check_chunk_range()


def test_fallback_with_grad_raises():
    sorernn_amd.set_range_guard("fallback")
    d = _inputs(BIG).to(DEV)
    q = d.q.clone().requires_grad_(True)
    with pytest.raises(FloatingPointError, match="backward"):
        chunk_gated_delta_rule(q, d.k, d.v, d.g, d.beta, scale=d.scale, initial_state=d.h0)


def test_noalloc_entry_sets_the_same_flag():
    sorernn_amd.set_range_guard("warn")
    _run(_inputs())  # registers the flag word of this device
    sorernn_amd.check_chunk_range()
    inp = _inputs(BIG, seed=71)
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
    _run(_inputs(BIG))
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
