"""GPU: the chunked forward with the layer's gated RMSNorm in the same call
(``chunk_gated_delta_rule_gated_norm``, ``gdn_chunk_fwd_gated_norm``) against the two-op route it
replaces -- ``chunk_gated_delta_rule`` then ``rms_norm_gated`` (sore/model/gdn.py:166-169 then
182-186), or ``o_norm(o) * F.silu(gate)`` with ``norm_split`` (gdn.py:188) -- and against the CPU
oracle's rule followed by the oracle norm.

The call takes one of two routes. When the chains' V / 32 column slices leave at least two CUs
per chain free, epilogue workgroups of the same launch normalise each O tile once all its slices
have stored it (progress words); otherwise the norm kernel follows the chunk kernel in place. Both
use the norm kernel's arithmetic, so the output equals the two-op route's bit for bit (with
``norm_split`` the silu(gate) rounding of torch's F.silu may differ by one bf16 step). The cases
cover several slices per head (V = 128), two (V = 64), grouped value heads, varlen documents that
end inside a chunk, the kernel's gate and beta options, the BASELINE config-4 layer size (epilogue
workgroups), many chains (in place, including the persistent grid of many documents) and the
layer's inference route with its ``fused_epilogue`` switch on. The oracle bar is max-abs 2e-2 of
the normalised output's scale.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import recurrent_gated_delta_rule, rms_norm, rms_norm_gated
from sorernn_amd import chunk_gated_delta_rule, chunk_gated_delta_rule_gated_norm
from sorernn_amd import rms_norm_gated as gpu_rms_norm_gated
from sorernn_amd.synthetic import gdn_inputs
from tests.parity import assert_output_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-6


def _gate_weight(shape, vd, seed):
    gen = torch.Generator().manual_seed(seed)
    gate = torch.randn(*shape, generator=gen).to(torch.bfloat16)
    w = 1.0 + 0.1 * torch.randn(vd, generator=gen)
    return gate, w


def _both(inp, gate, w, split, **kw):
    d = inp.to(DEV)
    gd, wd = gate.to(DEV), w.to(DEV)
    common = dict(scale=inp.scale, initial_state=d.h0, output_final_state=True, cu_seqlens=d.cu_seqlens,
                  cu_seqlens_cpu=inp.cu_seqlens, **kw)
    y, st = chunk_gated_delta_rule_gated_norm(d.q, d.k, d.v, d.g, d.beta, gd, wd, EPS, norm_split=split, **common)
    o, st2 = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, **common)
    if split:
        y2 = gpu_rms_norm_gated(o, None, wd, None, eps=EPS) * F.silu(gd)
    else:
        y2 = gpu_rms_norm_gated(o, gd, wd, None, activation="swish", eps=EPS)
    torch.cuda.synchronize()
    return y.cpu(), st.cpu(), y2.cpu(), st2.cpu()


def _oracle(inp, gate, w, split):
    cu = None if inp.cu_seqlens is None else inp.cu_seqlens.long()
    o, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True, cu_seqlens=cu)
    if split:
        return (rms_norm(o, w, EPS).to(torch.bfloat16).float() * F.silu(gate.float()).to(torch.bfloat16).float())
    return rms_norm_gated(o, gate, w, EPS)


def _epilogue_route(n, hv, vd):
    """True when the call runs its norm in epilogue workgroups (the host's rule)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return n * hv * (vd // 32) + 2 * n * hv <= cus


def _same_as_two_op(y, y2, split):
    if not split:
        assert torch.equal(y, y2), f"fused vs two-op max diff {(y.float() - y2.float()).abs().max().item():.3e}"
        return
    # torch's F.silu(gate) against the kernel's silu: one bf16 rounding step of the output at most
    diff = (y.float() - y2.float()).abs()
    assert (diff <= y2.float().abs() * 2.0 ** -7 + 1e-3).all(), f"fused vs two-op max diff {diff.max().item():.3e}"


def _check(y, st, y2, st2, ref, split=False):
    assert torch.isfinite(y).all()
    assert torch.equal(st, st2), "the final state is the plain call's"
    _same_as_two_op(y, y2, split)
    assert_output_close(y, ref, tol=2e-2 * float(ref.abs().max()))


@pytest.mark.parametrize("split", [False, True], ids=["fused_round", "split_round"])
@pytest.mark.parametrize("dims", [(128, 128, 2), (64, 64, 1), (128, 128, 1)], ids=["d128_gva2x", "d64", "d128"])
def test_fused_norm_matches_two_op_route(split, dims):
    kd, vd, rep = dims
    print(f"fused norm K={kd} V={vd} rep={rep} split={split}", flush=True)
    inp = gdn_inputs(2, 300, 2, kd, V=vd, HV=2 * rep, dtype=torch.bfloat16, seed=40 + kd + rep, h0=True)
    gate, w = _gate_weight(inp.v.shape, vd, 5)
    assert _epilogue_route(2, 2 * rep, vd)
    _check(*_both(inp, gate, w, split), _oracle(inp, gate, w, split), split)


def test_fused_norm_varlen_documents():
    cu = torch.tensor([0, 1, 63, 64, 200, 777], dtype=torch.long)
    inp = gdn_inputs(1, 777, 2, 128, HV=4, dtype=torch.bfloat16, seed=48, h0=True, cu_seqlens=cu)
    gate, w = _gate_weight(inp.v.shape, 128, 6)
    _check(*_both(inp, gate, w, False), _oracle(inp, gate, w, False))


def test_fused_norm_kernel_options():
    """Unnormalised q/k, gate and beta logits as the layer passes them with gdn_kernel_gate."""
    gen = torch.Generator().manual_seed(49)
    t, h, hv, dd = 257, 2, 4, 128
    q = (torch.randn(1, t, h, dd, generator=gen) * 2).to(torch.bfloat16)
    k = (torch.randn(1, t, h, dd, generator=gen) * 2).to(torch.bfloat16)
    v = torch.randn(1, t, hv, dd, generator=gen).to(torch.bfloat16)
    a = torch.randn(1, t, hv, generator=gen).to(torch.bfloat16)
    bl = torch.randn(1, t, hv, generator=gen).to(torch.bfloat16)
    A_log = torch.rand(hv, generator=gen) * 2
    dt_bias = torch.randn(hv, generator=gen) * 0.5
    gate, w = _gate_weight(v.shape, dd, 7)
    d = [x.to(DEV) for x in (q, k, v, a, bl, gate, w, A_log, dt_bias)]
    kw = dict(scale=dd ** -0.5, use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
              use_gate_in_kernel=True, A_log=d[7], dt_bias=d[8])
    y, _ = chunk_gated_delta_rule_gated_norm(d[0], d[1], d[2], d[3], d[4], d[5], d[6], EPS, **kw)
    o, _ = chunk_gated_delta_rule(d[0], d[1], d[2], d[3], d[4], **kw)
    y2 = gpu_rms_norm_gated(o, d[5], d[6], None, activation="swish", eps=EPS)
    torch.cuda.synchronize()
    _same_as_two_op(y.cpu(), y2.cpu(), False)


def test_fused_norm_config4_size():
    """BASELINE config 4's GDN call (B=2, T=8192, H=16, d=128), against the two-op route in full."""
    print("fused norm config-4 size", flush=True)
    inp = gdn_inputs(2, 8192, 16, 128, dtype=torch.bfloat16, seed=50, h0=False)
    gate, w = _gate_weight(inp.v.shape, 128, 8)
    assert _epilogue_route(2, 16, 128)
    y, st, y2, st2 = _both(inp, gate, w, False)
    assert torch.isfinite(y).all() and torch.equal(st, st2)
    _same_as_two_op(y, y2, False)


@pytest.mark.parametrize("split", [False, True], ids=["fused_round", "split_round"])
def test_fused_norm_in_place_route_many_chains(split):
    """Config 1's shape (64 chains, 256 slices: no CU left for epilogue workgroups): the chunk kernel
    stores O into the output and the norm kernel follows in place."""
    print(f"fused norm in place, config-1 shape, split={split}", flush=True)
    inp = gdn_inputs(4, 4096, 16, 128, dtype=torch.bfloat16, seed=52, h0=True)
    assert not _epilogue_route(4, 16, 128)
    gate, w = _gate_weight(inp.v.shape, 128, 9)
    y, st, y2, st2 = _both(inp, gate, w, split)
    assert torch.isfinite(y).all() and torch.equal(st, st2)
    _same_as_two_op(y, y2, split)


def test_fused_norm_in_place_route_persistent_grid():
    """Many documents without initial or final state: the chunk call takes the persistent grid, then
    the norm kernel runs in place. Against the two-op route and the oracle."""
    gen = torch.Generator().manual_seed(53)
    lens = torch.randint(1, 200, (120,), generator=gen).tolist()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist())
    print(f"fused norm in place, persistent grid: {len(lens)} docs, {int(cu[-1])} tokens", flush=True)
    inp = gdn_inputs(1, int(cu[-1]), 2, 128, HV=4, dtype=torch.bfloat16, seed=54, cu_seqlens=cu)
    assert not _epilogue_route(len(lens), 4, 128)
    gate, w = _gate_weight(inp.v.shape, 128, 10)
    d = inp.to(DEV)
    gd, wd = gate.to(DEV), w.to(DEV)
    kw = dict(scale=inp.scale, cu_seqlens=d.cu_seqlens, cu_seqlens_cpu=inp.cu_seqlens)
    y, _ = chunk_gated_delta_rule_gated_norm(d.q, d.k, d.v, d.g, d.beta, gd, wd, EPS, **kw)
    o, _ = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, **kw)
    y2 = gpu_rms_norm_gated(o, gd, wd, None, activation="swish", eps=EPS)
    torch.cuda.synchronize()
    _same_as_two_op(y.cpu(), y2.cpu(), False)
    o_ref, _ = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, None, False,
                                          cu_seqlens=cu.long())
    ref = rms_norm_gated(o_ref, gate, w, EPS)
    assert_output_close(y.cpu(), ref, tol=2e-2 * float(ref.abs().max()))


def test_fused_norm_epilogue_many_documents_with_states():
    """Epilogue workgroups over 12 documents of 1-700 tokens at HV = 2 (24 chains, shared chains and
    chunk strides), with initial and final states, against the two-op route and the oracle."""
    gen = torch.Generator().manual_seed(55)
    lens = torch.randint(1, 700, (12,), generator=gen).tolist()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist())
    inp = gdn_inputs(1, int(cu[-1]), 2, 128, HV=2, dtype=torch.bfloat16, seed=56, h0=True, cu_seqlens=cu)
    assert _epilogue_route(12, 2, 128)
    gate, w = _gate_weight(inp.v.shape, 128, 11)
    _check(*_both(inp, gate, w, False), _oracle(inp, gate, w, False))


def test_fused_norm_l2norm_on_few_long_chains():
    """use_qk_l2norm_in_kernel on a few-chain call (one 4096-token sequence, 4 value heads): the op
    normalises q and k with the row kernel first and runs the fused kernel without the flag. Against
    the oracle (F.normalize then the rule and the norm) and the two-op route on the same raw q/k."""
    from sorernn_amd.ops import _l2norm_first

    gen = torch.Generator().manual_seed(41)
    t, h, hv, dd = 4096, 2, 4, 128
    q = (torch.randn(1, t, h, dd, generator=gen) * 3).to(torch.bfloat16)
    k = (torch.randn(1, t, h, dd, generator=gen) * 3).to(torch.bfloat16)
    v = torch.randn(1, t, hv, dd, generator=gen).to(torch.bfloat16)
    g = -F.softplus(torch.randn(1, t, hv, generator=gen))
    beta = torch.rand(1, t, hv, generator=gen)
    gate, w = _gate_weight(v.shape, dd, 42)
    d = [x.to(DEV) for x in (q, k, v, g, beta, gate, w)]
    assert _l2norm_first(d[0], 1, hv, dd, t)
    y, _ = chunk_gated_delta_rule_gated_norm(d[0], d[1], d[2], d[3], d[4], d[5], d[6], EPS, scale=dd**-0.5,
                                             use_qk_l2norm_in_kernel=True)
    o, _ = chunk_gated_delta_rule(d[0], d[1], d[2], d[3], d[4], scale=dd**-0.5, use_qk_l2norm_in_kernel=True)
    y2 = gpu_rms_norm_gated(o, d[5], d[6], None, activation="swish", eps=EPS)
    torch.cuda.synchronize()
    diff = (y.float() - y2.float()).abs()
    assert (diff <= y2.float().abs() * 2.0 ** -7 + 1e-3).all(), f"fused vs two-op max diff {diff.max().item():.3e}"
    qn = F.normalize(q.float(), dim=-1).to(torch.bfloat16)
    kn = F.normalize(k.float(), dim=-1).to(torch.bfloat16)
    o_ref, _ = recurrent_gated_delta_rule(qn, kn, v, g, beta, dd**-0.5, None, False)
    ref = rms_norm_gated(o_ref, gate, w, EPS)
    assert_output_close(y.cpu(), ref, tol=2e-2 * float(ref.abs().max()))


def test_fused_norm_rejects_grad():
    inp = gdn_inputs(1, 64, 2, 128, dtype=torch.bfloat16, seed=51)
    d = inp.to(DEV)
    gate, w = _gate_weight(inp.v.shape, 128, 9)
    q = d.q.clone().requires_grad_(True)
    with pytest.raises(NotImplementedError, match="inference only"):
        chunk_gated_delta_rule_gated_norm(q, d.k, d.v, d.g, d.beta, gate.to(DEV), w.to(DEV), EPS)


@pytest.mark.parametrize("fused_norm_gate", [True, False], ids=["fused_flag", "unfused_flag"])
@pytest.mark.parametrize("cu_case", ["rows", "short_docs"])
def test_layer_with_fused_epilogue_matches_oracle(fused_norm_gate, cu_case, monkeypatch):
    """The layer's inference route with ``fused_epilogue`` on (the norm inside the chunk kernel, both
    rounding routes of fused_norm_gate) against the layer oracle; the norm kernel is not called."""
    from tests.test_gpu_layer import _CU_CASES, _layer, _oracle_forward, _run
    import sorernn_amd.gdn_layer as gl

    cu = _CU_CASES[cu_case]
    layer = _layer(True, rep=2, fla_conv=True, fused_norm_gate=fused_norm_gate)
    b = 2 if cu is None else 1
    x = torch.randn(b, 512, 256, generator=torch.Generator().manual_seed(13))
    cu_t = None if cu is None else torch.tensor(cu)
    ref = _oracle_forward(layer, x, cu_t)
    layer = layer.to(DEV)
    layer.fused_epilogue = True

    def no_norm_kernel(*a, **k):
        raise AssertionError("the fused epilogue route called the separate norm kernel")

    monkeypatch.setattr(gl, "rms_norm_gated", no_norm_kernel)
    out = _run(layer, x, cu_t)
    err = (out - ref).abs().max().item()
    assert err <= 2e-2 * ref.abs().max().item() + 1e-3, f"max-abs error {err:.3e} (max|ref| {ref.abs().max():.3e})"


@pytest.mark.parametrize("n_docs", [10, 100], ids=["epilogue_route", "in_place_route"])
def test_fused_norm_empty_sequences_through_the_abi(n_docs):
    """Empty sequences (allowed by the C ABI, rejected by the Python op as the reference's cu_seqlens
    contract does) on both routes, with initial and final states: the outputs equal the plain entry
    point's O normalised by the norm kernel, bit for bit, and the final states are the plain call's
    (an empty sequence's final state is its initial state)."""
    from sorernn_amd import _lib

    gen = torch.Generator().manual_seed(57 + n_docs)
    lens = torch.randint(1, 150, (n_docs,), generator=gen).tolist()
    for i in (0, n_docs // 2, n_docs - 1):
        lens[i] = 0
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist())
    t, n, hv = int(cu[-1]), n_docs, 4
    assert _epilogue_route(n, hv, 128) == (n_docs == 10)
    print(f"fused norm, empty sequences through the ABI: {n} docs, {t} tokens", flush=True)
    inp = gdn_inputs(1, t, 2, 128, HV=hv, dtype=torch.bfloat16, seed=58, h0=True, cu_seqlens=cu)
    gate, w = _gate_weight(inp.v.shape, 128, 12)
    d = inp.to(DEV)
    gd, wd = gate.to(DEV), w.to(DEV)
    lib = _lib.load()
    common = [_lib.ptr(d.q), _lib.ptr(d.k), _lib.ptr(d.v), _lib.ptr(d.g), _lib.ptr(d.beta), _lib.ptr(d.h0)]
    sizes = [1, t, 2, hv, 128, 128, n, _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32, inp.scale, 0, None, None]
    y = torch.empty(1, t, hv, 128, device=DEV, dtype=torch.bfloat16)
    st = torch.empty(n, hv, 128, 128, device=DEV, dtype=torch.float32)
    nb = int(lib.gdn_chunk_gated_norm_workspace_size(1, t, hv, n, 128, 1))
    ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
    _lib.call("gdn_chunk_fwd_gated_norm", *common, _lib.ptr(y), _lib.ptr(st), _lib.ptr(d.cu_seqlens), *sizes,
              _lib.ptr(gd), _lib.ptr(wd), EPS, 0, _lib.ptr(ws), nb, _lib.stream_of(d.q))
    o = torch.empty_like(y)
    st2 = torch.empty_like(st)
    nb2 = int(lib.gdn_chunk_workspace_size(1, t, hv, n, 1))
    ws2 = torch.empty(nb2, dtype=torch.uint8, device=DEV)
    _lib.call("gdn_chunk_fwd", *common, _lib.ptr(o), _lib.ptr(st2), _lib.ptr(d.cu_seqlens), *sizes, _lib.ptr(ws2), nb2,
              _lib.stream_of(d.q))
    y2 = gpu_rms_norm_gated(o, gd, wd, None, activation="swish", eps=EPS)
    torch.cuda.synchronize()
    _same_as_two_op(y.cpu(), y2.cpu(), False)
    assert torch.equal(st.cpu(), st2.cpu())
    for i in (0, n_docs // 2, n_docs - 1):
        assert torch.equal(st[i].cpu(), inp.h0[i]), f"empty sequence {i}: final state is not its initial state"


@pytest.mark.parametrize("varlen", [False, True], ids=["fixed", "varlen"])
def test_fused_norm_fp16_overflow_is_recomputed(varlen):
    """v x 1e5 on the epilogue route: the chunk kernel's fp16 operands overflow while the fp32
    results stay finite (tests/test_gpu_range.py). A slice that stored a non-finite O publishes no
    chunk from that one on, recomputes its columns in fp32, and publishes them afterwards: y is
    finite and meets the oracle's bar (the RMS norm removes the input's scale), the final states
    equal the plain call's, and the range flag stays clear."""
    import sorernn_amd

    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    big = 1.0e5
    if varlen:
        cu = torch.tensor([0, 40, 41, 300], dtype=torch.long)
        inp = gdn_inputs(1, 300, 2, 128, HV=4, dtype=torch.bfloat16, seed=72, h0=True, cu_seqlens=cu)
        n, hv = 3, 4
    else:
        inp = gdn_inputs(1, 130, 2, 128, dtype=torch.bfloat16, seed=70, h0=True)
        n, hv = 1, 2
    inp.v = (inp.v.float() * big).to(torch.bfloat16)
    assert _epilogue_route(n, hv, 128)
    print(f"fused norm, v x {big:g}, varlen={varlen}", flush=True)
    gate, w = _gate_weight(inp.v.shape, 128, 13)
    y, st, y2, st2 = _both(inp, gate, w, False)
    assert torch.isfinite(y).all() and torch.isfinite(st).all()
    assert torch.equal(st, st2), "the final state is the plain call's (both recomputed in fp32)"
    ref = _oracle(inp, gate, w, False)
    scale = float(ref.abs().max())
    assert_output_close(y, ref, tol=2e-2 * scale)
    assert (y.float() - y2.float()).abs().max().item() <= 2e-2 * scale
    assert not sorernn_amd.check_chunk_range(), "the recomputation was finite: the flag must stay clear"


def test_fused_norm_two_streams_at_once():
    """Two calls on the epilogue route issued on two streams at once, each grid as large as the
    machine: the slices never wait for the epilogue workgroups, and each launch dispatches its
    slices first, so both complete; each output equals the same call run alone."""
    import sorernn_amd

    sorernn_amd.set_range_guard("warn")
    sorernn_amd.check_chunk_range()
    runs = []
    for seed in (60, 61):
        inp = gdn_inputs(2, 1024, 4, 128, dtype=torch.bfloat16, seed=seed, h0=True)
        gate, w = _gate_weight(inp.v.shape, 128, seed)
        runs.append((inp.to(DEV), gate.to(DEV), w.to(DEV), inp.scale))
    assert _epilogue_route(2, 4, 128)

    def call(r):
        d, gd, wd, sc = r
        return chunk_gated_delta_rule_gated_norm(d.q, d.k, d.v, d.g, d.beta, gd, wd, EPS, scale=sc,
                                                 initial_state=d.h0, output_final_state=True)

    alone = [call(r) for r in runs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    for s, r in zip(streams, runs):
        with torch.cuda.stream(s):
            outs.append(call(r))
    torch.cuda.synchronize()
    for (y, st), (y0, st0) in zip(outs, alone):
        assert torch.equal(y, y0) and torch.equal(st, st0)
    assert not sorernn_amd.check_chunk_range(), "a wait ran out"
