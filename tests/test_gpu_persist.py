"""GPU parity of the persistent chunk grid (``chunk_gated_delta_rule`` with cu_seqlens and many chains).

When a varlen inference call without initial or final states (the reference model's call,
sore/model/gdn.py:166-169) has at least four (sequence, value head) chains per group of workgroups
(groups = CUs / (V / 32); 64 on MI355X at V = 128), the state kernel runs one workgroup per CU and
each group walks a job list of chains, its pipeline continuing from one chain into the next. These
tests check it against the oracle (one-token documents, GVA, K/V 64 and 128, the in-kernel gate
options, empty sequences through the C ABI, fp16 overflow recovery, the reference's document lengths
at full size, and both schedulers: LPT by rows of HV groups, and snake order for more than 128
sequences or a head count that does not divide the group count) and, per document, bitwise against
the same document run alone (one chain per workgroup: the non-persistent grid), since each chain's
arithmetic is the same on both. A many-chain call with states takes the non-persistent grid and is checked against the
oracle too. Tolerances: max-abs 2e-2 on bf16 outputs, relative L2 1e-3 on fp32 final states.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import recurrent_gated_delta_rule
from sorernn_amd import chunk_gated_delta_rule
from sorernn_amd.synthetic import gdn_inputs
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lengths(n, lo, hi, seed, extra=()):
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n - len(extra),), generator=gen).tolist() + list(extra)
    perm = torch.randperm(n, generator=gen).tolist()
    return [lens[i] for i in perm]


def _cu(lens):
    return torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.long)


def _run(inp, states=False, **kw):
    d = inp.to(DEV)
    o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0 if states else None,
                                   output_final_state=states, cu_seqlens=d.cu_seqlens, cu_seqlens_cpu=inp.cu_seqlens,
                                   **kw)
    torch.cuda.synchronize()
    return o, st


@pytest.mark.parametrize("kv", [(128, 128), (64, 64), (128, 64)], ids=lambda x: f"K{x[0]}V{x[1]}")
def test_persistent_grid_matches_oracle(kv):
    kd, vd = kv
    docs = 64 if vd == 128 else 128  # four chains per group at HV = 4
    lens = _lengths(docs, 1, 260, seed=kd + vd, extra=(1, 1, 64, 65, 700))
    cu = _cu(lens)
    print(f"persistent K={kd} V={vd}: {docs} docs, {int(cu[-1])} tokens", flush=True)
    inp = gdn_inputs(1, int(cu[-1]), 2, kd, V=vd, HV=4, dtype=torch.bfloat16, seed=51, h0=True, cu_seqlens=cu)
    o, st = _run(inp)
    assert st is None
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, None, False, cu_seqlens=cu)
    assert_output_close(o.cpu(), o_ref)


def test_many_chains_with_states_keep_the_slice_grid():
    """The same many-chain shape with initial and final states (one workgroup per slice)."""
    lens = _lengths(64, 1, 260, seed=5, extra=(1, 64, 65, 700))
    cu = _cu(lens)
    inp = gdn_inputs(1, int(cu[-1]), 2, 128, HV=4, dtype=torch.bfloat16, seed=55, h0=True, cu_seqlens=cu)
    o, st = _run(inp, states=True)
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True,
                                               cu_seqlens=cu)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)


def test_persistent_grid_empty_sequences_through_the_abi():
    """Empty sequences (which chunk_gated_delta_rule rejects, as the reference's cu_seqlens contract
    does) are in no job list; through the C ABI the other sequences are unaffected."""
    from sorernn_amd import _lib
    from sorernn_amd.ops import chunk_workspace_bytes

    lens = _lengths(64, 1, 200, seed=11, extra=(0, 0, 0))
    cu = _cu(lens)
    t = int(cu[-1])
    print(f"persistent empty sequences: {t} tokens", flush=True)
    inp = gdn_inputs(1, t, 2, 128, HV=4, dtype=torch.bfloat16, seed=54, h0=True, cu_seqlens=cu)
    d = inp.to(DEV)
    n = len(lens)
    o = torch.empty(1, t, 4, 128, device=DEV, dtype=torch.bfloat16)
    nbytes = chunk_workspace_bytes(1, t, 4, n, True)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    _lib.call("gdn_chunk_fwd", _lib.ptr(d.q), _lib.ptr(d.k), _lib.ptr(d.v), _lib.ptr(d.g), _lib.ptr(d.beta),
              None, _lib.ptr(o), None, _lib.ptr(d.cu_seqlens), 1, t, 2, 4, 128, 128, n,
              _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32, inp.scale, 0, None, None, _lib.ptr(ws), nbytes,
              _lib.stream_of(d.q))
    torch.cuda.synchronize()
    keep = [i for i, x in enumerate(lens) if x > 0]
    cu_ne = _cu([lens[i] for i in keep])
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, None, False,
                                          cu_seqlens=cu_ne)
    assert_output_close(o.cpu(), o_ref)


def test_persistent_grid_bitwise_equals_documents_alone():
    lens = _lengths(64, 20, 200, seed=7, extra=(1, 130))
    cu = _cu(lens)
    print(f"persistent vs alone: {int(cu[-1])} tokens", flush=True)
    inp = gdn_inputs(1, int(cu[-1]), 4, 128, HV=4, dtype=torch.bfloat16, seed=52, cu_seqlens=cu)
    o, _ = _run(inp)
    for i in sorted(range(64), key=lambda j: -lens[j])[:3] + [lens.index(1), lens.index(130)]:
        a, b = int(cu[i]), int(cu[i + 1])
        one = type(inp)(inp.q[:, a:b].contiguous(), inp.k[:, a:b].contiguous(), inp.v[:, a:b].contiguous(),
                        inp.g[:, a:b].contiguous(), inp.beta[:, a:b].contiguous(), None, None, inp.scale)
        o1, _ = _run(one)
        assert torch.equal(o1, o[:, a:b]), f"document {i}: o differs from the document run alone"


def test_persistent_grid_zero_state_and_kernel_options():
    """The reference model's call: no initial state, no final state; the in-kernel gate, beta sigmoid
    and q/k L2 norm (A_log and dt_bias per value head, read per job)."""
    lens = _lengths(64, 1, 300, seed=9)
    cu = _cu(lens)
    t, h, hv, d = int(cu[-1]), 2, 4, 128
    print(f"persistent kernel options: {t} tokens", flush=True)
    gen = torch.Generator().manual_seed(53)
    q = (torch.randn(1, t, h, d, generator=gen) * 2).to(torch.bfloat16)
    k = (torch.randn(1, t, h, d, generator=gen) * 2).to(torch.bfloat16)
    v = torch.randn(1, t, hv, d, generator=gen).to(torch.bfloat16)
    a = torch.randn(1, t, hv, generator=gen).to(torch.bfloat16)
    b = torch.randn(1, t, hv, generator=gen).to(torch.bfloat16)
    A_log = torch.empty(hv).uniform_(1, 16, generator=gen).log()
    dt_bias = torch.randn(hv, generator=gen) * 0.3
    dev = lambda x: x.to(DEV)  # noqa: E731
    o, fin = chunk_gated_delta_rule(dev(q), dev(k), dev(v), dev(a), dev(b), output_final_state=False,
                                    use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                                    use_gate_in_kernel=True, A_log=dev(A_log), dt_bias=dev(dt_bias),
                                    cu_seqlens=dev(cu), cu_seqlens_cpu=cu)
    torch.cuda.synchronize()
    assert fin is None
    g_ref = -A_log.exp() * F.softplus(a.float() + dt_bias)
    qn = F.normalize(q.float(), dim=-1).to(torch.bfloat16)
    kn = F.normalize(k.float(), dim=-1).to(torch.bfloat16)
    o_ref, _ = recurrent_gated_delta_rule(qn, kn, v, g_ref, b.float().sigmoid(), d**-0.5, None, False, cu_seqlens=cu)
    assert_output_close(o.cpu(), o_ref)


def test_persistent_grid_recomputes_fp16_overflow():
    """v x 1e5 (past the fp16 range of the matrix-core operands): a workgroup of the persistent grid
    that stored an inf/NaN recomputes its V-slice of every job in its list by the fp32 recurrence, so
    the outputs are finite and meet the bars at the input's scale; the range flag stays clear."""
    import sorernn_amd

    big = 1.0e5
    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    lens = _lengths(64, 1, 200, seed=13, extra=(1, 130))
    cu = _cu(lens)
    print(f"persistent v x {big:g}: {int(cu[-1])} tokens", flush=True)
    inp = gdn_inputs(1, int(cu[-1]), 2, 128, HV=4, dtype=torch.bfloat16, seed=56, cu_seqlens=cu)
    inp.v = (inp.v.float() * big).to(torch.bfloat16)
    o, _ = _run(inp)
    assert torch.isfinite(o).all()
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, None, False, cu_seqlens=cu)
    assert_output_close((o.float().cpu() / big).to(torch.bfloat16), o_ref.float() / big, what="o / 1e5")
    assert not sorernn_amd.check_chunk_range()


def test_persistent_grid_reference_document_lengths_full_size():
    """The bench's real-distribution workload at full size (53 documents of the reference's corpus
    lengths in 32,768 tokens, HV = 16: rows of 16 groups, scheduled with the row loads in scalar
    registers), checked on the longest, a mid-length and the shortest document, two value heads each."""
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "doc_lengths_pt.json")
    with open(path) as f:
        lens = [n for w in json.load(f)["windows"] for n in w]
    cu = _cu(lens)
    print(f"persistent reference lengths: {len(lens)} docs, {int(cu[-1])} tokens", flush=True)
    inp = gdn_inputs(1, int(cu[-1]), 16, 128, dtype=torch.bfloat16, seed=57, cu_seqlens=cu)
    o, _ = _run(inp)
    o = o.cpu()
    heads = [0, 13]
    srt = sorted(range(len(lens)), key=lambda i: lens[i])
    for n in (srt[-1], srt[len(srt) // 2], srt[0]):
        a, e = int(cu[n]), int(cu[n + 1])
        sl = lambda x: x[:, a:e, heads]  # noqa: E731
        o_ref, _ = recurrent_gated_delta_rule(sl(inp.q), sl(inp.k), sl(inp.v), sl(inp.g), sl(inp.beta), inp.scale,
                                              None, False)
        assert_output_close(o[:, a:e, heads], o_ref, what=f"o of document {n} ({lens[n]} tokens)")


@pytest.mark.parametrize("shape", [(200, 1, 4), (100, 1, 3)], ids=["over_128_sequences", "hv3_snake"])
def test_persistent_grid_snake_order(shape):
    """Job lists in snake order: more sequences than the LPT scheduler takes (200 > 128), or a head
    count that does not divide the group count (HV = 3, 64 groups); short documents, GVA."""
    docs, h, hv = shape
    lens = _lengths(docs, 1, 90, seed=docs + hv, extra=(1, 64, 65))
    cu = _cu(lens)
    print(f"persistent snake order: {docs} docs, HV={hv}, {int(cu[-1])} tokens", flush=True)
    inp = gdn_inputs(1, int(cu[-1]), h, 128, HV=hv, dtype=torch.bfloat16, seed=58, cu_seqlens=cu)
    o, _ = _run(inp)
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, None, False, cu_seqlens=cu)
    assert_output_close(o.cpu(), o_ref)
