"""GPU parity of the fused chunked prefill kernel (``chunk_gated_delta_rule``) vs the CPU oracle.

Small shapes compare against the oracle directly; the BASELINE config-1 size is compared against
the oracle on a slice (one batch row, two heads, all 4096 tokens) and, in full, against the GPU
recurrent kernel (exact fp32 token-by-token path), plus split invariance at full length.
Tolerances: max-abs 2e-2 on bf16 outputs, relative L2 1e-3 on fp32 final states.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import recurrent_gated_delta_rule
from sorernn_amd import _lib, chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
from sorernn_amd.synthetic import config_inputs, gdn_inputs, varlen_cu_seqlens
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _chunk(inp, **kw):
    d = inp.to(DEV)
    o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                   output_final_state=True, cu_seqlens=d.cu_seqlens,
                                   cu_seqlens_cpu=inp.cu_seqlens, **kw)
    torch.cuda.synchronize()
    return o, st


def _oracle(inp):
    cu = None if inp.cu_seqlens is None else inp.cu_seqlens.long()
    return recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True, cu_seqlens=cu)


@pytest.mark.parametrize("t", [256, 200, 65, 64, 1], ids=lambda t: f"T{t}")
@pytest.mark.parametrize("h0", [False, True], ids=["zero_h0", "h0"])
def test_chunk_small_matches_oracle(t, h0):
    print(f"chunk T={t} h0={h0}", flush=True)
    inp = gdn_inputs(1, t, 4, 64, dtype=torch.bfloat16, seed=1000, h0=h0)
    o, st = _chunk(inp)
    o_ref, st_ref = _oracle(inp)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)


@pytest.mark.parametrize("kv", [(128, 128), (64, 64), (128, 64), (64, 128)], ids=lambda x: f"K{x[0]}V{x[1]}")
def test_chunk_head_dims(kv):
    kd, vd = kv
    print(f"chunk K={kd} V={vd}", flush=True)
    inp = gdn_inputs(2, 300, 3, kd, V=vd, dtype=torch.bfloat16, seed=7, h0=True)
    o, st = _chunk(inp)
    o_ref, st_ref = _oracle(inp)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)


@pytest.mark.parametrize("cu", [[0, 1, 3, 4, 70, 200, 512], [0, 512], [0, 63, 64, 65, 129, 300]],
                         ids=["short_docs", "one_doc", "chunk_edges"])
@pytest.mark.parametrize("rep", [1, 2], ids=["no_gva", "gva2x"])
def test_chunk_varlen_matches_oracle(cu, rep):
    print(f"chunk varlen cu={cu} rep={rep}", flush=True)
    cu_t = torch.tensor(cu, dtype=torch.long)
    inp = gdn_inputs(1, cu[-1], 2, 128, HV=2 * rep, dtype=torch.bfloat16, seed=3, h0=True, cu_seqlens=cu_t)
    o, st = _chunk(inp)
    o_ref, st_ref = _oracle(inp)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)


def test_chunk_kernel_options_match_oracle():
    # raw inputs as sore/model/gdn.py passes them with gdn_kernel_gate: unnormalised q/k, a, b logits
    gen = torch.Generator().manual_seed(31)
    t, h, hv, d = 200, 2, 4, 128
    q = (torch.randn(1, t, h, d, generator=gen) * 2).to(torch.bfloat16)
    k = (torch.randn(1, t, h, d, generator=gen) * 2).to(torch.bfloat16)
    v = torch.randn(1, t, hv, d, generator=gen).to(torch.bfloat16)
    a = torch.randn(1, t, hv, generator=gen).to(torch.bfloat16)
    b = torch.randn(1, t, hv, generator=gen).to(torch.bfloat16)
    A_log = torch.empty(hv).uniform_(1, 16, generator=gen).log()
    dt_bias = torch.randn(hv, generator=gen) * 0.3
    cu = torch.tensor([0, 5, 77, 200])
    dev = lambda x: x.to(DEV)  # noqa: E731
    o, st = chunk_gated_delta_rule(dev(q), dev(k), dev(v), dev(a), dev(b), initial_state=None, output_final_state=True,
                                   use_qk_l2norm_in_kernel=True, use_beta_sigmoid_in_kernel=True,
                                   use_gate_in_kernel=True, A_log=dev(A_log), dt_bias=dev(dt_bias),
                                   cu_seqlens=dev(cu), cu_seqlens_cpu=cu)
    g_ref = -A_log.exp() * F.softplus(a.float() + dt_bias)
    qn = F.normalize(q.float(), dim=-1).to(torch.bfloat16)
    kn = F.normalize(k.float(), dim=-1).to(torch.bfloat16)
    o_ref, st_ref = recurrent_gated_delta_rule(qn, kn, v, g_ref, b.float().sigmoid(), d**-0.5, None, True, cu_seqlens=cu)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)


def test_chunk_kernel_in_kernel_l2norm_through_the_abi():
    """The two q/k L2-norm routes of an inference call: inside the chunk kernels
    (GDN_FLAG_QK_L2NORM through gdn_chunk_fwd, as C callers, the training forward and calls that
    fill the chip use it), and the row kernel first with the flag cleared (the Python op's route for
    few, long chains: here one 4096-token sequence, 16 workgroups). Both against the oracle, and
    against each other within half the output bar (the routes sum the squares in a different order,
    so a normalised element can differ by one bf16 step)."""
    from sorernn_amd.ops import _l2norm_first, chunk_workspace_bytes

    gen = torch.Generator().manual_seed(33)
    t, h, hv, d = 4096, 2, 4, 128
    q = (torch.randn(1, t, h, d, generator=gen) * 3).to(torch.bfloat16)
    k = (torch.randn(1, t, h, d, generator=gen) * 3).to(torch.bfloat16)
    v = torch.randn(1, t, hv, d, generator=gen).to(torch.bfloat16)
    g = -F.softplus(torch.randn(1, t, hv, generator=gen))
    beta = torch.rand(1, t, hv, generator=gen)
    h0 = 0.02 * torch.randn(1, hv, d, d, generator=gen)
    qd, kd_, vd_, gd, bd, h0d = (x.to(DEV) for x in (q, k, v, g, beta, h0))
    assert _l2norm_first(qd, 1, hv, d, t), "this shape takes the row-kernel route"
    assert not _l2norm_first(qd, 4, 16, 128, 4 * 4096), "config 1 keeps the flag in the kernels"
    o = torch.empty(1, t, hv, d, device=DEV, dtype=torch.bfloat16)
    st = torch.empty(1, hv, d, d, device=DEV)
    nbytes = chunk_workspace_bytes(1, t, hv, 1, False)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    _lib.call("gdn_chunk_fwd", _lib.ptr(qd), _lib.ptr(kd_), _lib.ptr(vd_), _lib.ptr(gd), _lib.ptr(bd), _lib.ptr(h0d),
              _lib.ptr(o), _lib.ptr(st), None, 1, t, h, hv, d, d, 1, _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32,
              d**-0.5, _lib.FLAG_QK_L2NORM, None, None, _lib.ptr(ws), nbytes, _lib.stream_of(qd))
    o_op, st_op = chunk_gated_delta_rule(qd, kd_, vd_, gd, bd, initial_state=h0d, output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    qn = F.normalize(q.float(), dim=-1).to(torch.bfloat16)
    kn = F.normalize(k.float(), dim=-1).to(torch.bfloat16)
    o_ref, st_ref = recurrent_gated_delta_rule(qn, kn, v, g, beta, d**-0.5, h0, True)
    assert_output_close(o.cpu(), o_ref, what="o (in-kernel L2 norm)")
    assert_state_close(st.cpu(), st_ref, what="final state (in-kernel L2 norm)")
    assert_output_close(o_op.cpu(), o_ref, what="o (row-kernel L2 norm)")
    assert_state_close(st_op.cpu(), st_ref, what="final state (row-kernel L2 norm)")
    diff = (o.float() - o_op.float()).abs().max().item()
    assert diff <= 1e-2, f"the two L2-norm routes differ by {diff:.3e}"


def test_chunk_in_kernel_gate_bf16_config1_size():
    """Regression for the state kernel's gate loads: raw bf16 a/b (the layer's gdn_kernel_gate route)
    at config-1 size. Each bf16 gate tensor is exactly 512 KiB; the last head of the last token is
    its final element, which the loads once read 2 bytes past. Checked against the oracle on a slice
    that holds that element (batch row 3, value heads 0 and 15, all 4096 tokens)."""
    print("config1 in-kernel gate, bf16 a/b", flush=True)
    inp = config_inputs(1)
    gen = torch.Generator().manual_seed(77)
    a = torch.randn(4, 4096, 16, generator=gen).to(torch.bfloat16)
    b = torch.randn(4, 4096, 16, generator=gen).to(torch.bfloat16)
    assert a.numel() * a.element_size() == 512 * 1024
    A_log = torch.empty(16).uniform_(1, 16, generator=gen).log()
    dt_bias = torch.randn(16, generator=gen) * 0.3
    d = inp.to(DEV)
    o, st = chunk_gated_delta_rule(d.q, d.k, d.v, a.to(DEV), b.to(DEV), scale=inp.scale, initial_state=d.h0,
                                   output_final_state=True, use_gate_in_kernel=True, A_log=A_log.to(DEV),
                                   dt_bias=dt_bias.to(DEV), use_beta_sigmoid_in_kernel=True)
    torch.cuda.synchronize()
    g_ref = -A_log.exp() * F.softplus(a.float() + dt_bias)
    sl = lambda x: x[3:4, :, [0, 15]]  # noqa: E731
    o_ref, st_ref = recurrent_gated_delta_rule(sl(inp.q), sl(inp.k), sl(inp.v), sl(g_ref), sl(b.float().sigmoid()),
                                               inp.scale, inp.h0[3:4, [0, 15]], True)
    assert_output_close(o[3:4, :, [0, 15]].cpu(), o_ref)
    assert_state_close(st[3:4, [0, 15]].cpu(), st_ref)


def test_chunk_matches_recurrent_kernel_config1_full_size():
    inp = config_inputs(1)
    print("config1 full size", flush=True)
    o, st = _chunk(inp)
    d = inp.to(DEV)
    o_r, st_r = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                                 output_final_state=True)
    torch.cuda.synchronize()
    assert_output_close(o, o_r.float())
    assert_state_close(st, st_r)
    # the oracle on a slice: batch row 1, heads 5 and 11, all 4096 tokens
    sl = lambda x: x[1:2, :, [5, 11]]  # noqa: E731
    o_ref, st_ref = recurrent_gated_delta_rule(sl(inp.q), sl(inp.k), sl(inp.v), sl(inp.g), sl(inp.beta), inp.scale,
                                               inp.h0[1:2, [5, 11]], True)
    assert_output_close(o[1:2, :, [5, 11]].cpu(), o_ref)
    assert_state_close(st[1:2, [5, 11]].cpu(), st_ref)


def test_chunk_split_invariance_config1():
    inp = config_inputs(1).to(DEV)
    kw = dict(scale=inp.scale, output_final_state=True)
    o, st = chunk_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, initial_state=inp.h0, **kw)
    t1 = 1000  # not a multiple of 64: the second call's chunks are shifted
    o1, s1 = chunk_gated_delta_rule(inp.q[:, :t1], inp.k[:, :t1], inp.v[:, :t1], inp.g[:, :t1], inp.beta[:, :t1],
                                    initial_state=inp.h0, **kw)
    o2, s2 = chunk_gated_delta_rule(inp.q[:, t1:], inp.k[:, t1:], inp.v[:, t1:], inp.g[:, t1:], inp.beta[:, t1:],
                                    initial_state=s1, **kw)
    assert_output_close(torch.cat([o1, o2], 1), o.float())
    assert_state_close(s2, st)


def test_chunk_varlen_config3_matches_recurrent_kernel():
    inp = config_inputs(3)
    print("config3 varlen", inp.cu_seqlens.tolist(), flush=True)
    o, st = _chunk(inp)
    d = inp.to(DEV)
    o_r, st_r = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                                 output_final_state=True, cu_seqlens=d.cu_seqlens,
                                                 cu_seqlens_cpu=inp.cu_seqlens)
    torch.cuda.synchronize()
    assert st.shape == (8, 16, 128, 128)
    assert_output_close(o, o_r.float())
    assert_state_close(st, st_r)


@pytest.mark.parametrize("varlen", [False, True], ids=["batched", "varlen"])
def test_tsolve_chunk_walk_covers_every_chunk(varlen):
    """The T-solve kernel's workgroups each solve several chunks of one value head in turn (stride =
    the grid's width). At 64 value heads and 102 chunks per head, a 256-CU device gets 15 workgroups
    per head, some walking 7 chunks and some 6, with a partial last chunk per sequence; with cu_seqlens
    the walk runs over an upper bound on the chunk count. Every output row and final state must match
    the GPU recurrent kernel (the exact fp32 token-by-token path)."""
    if varlen:
        gen = torch.Generator().manual_seed(7)
        lengths = (torch.randint(1, 400, (37,), generator=gen)).tolist()
        cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int64)
        inp = gdn_inputs(1, int(cu[-1]), 16, 64, HV=64, dtype=torch.bfloat16, seed=8, h0=True, n_states=37,
                         cu_seqlens=cu)
    else:
        inp = gdn_inputs(2, 3211, 16, 64, HV=64, dtype=torch.bfloat16, seed=8, h0=True)
    print("T-solve walk", "varlen" if varlen else "batched", tuple(inp.q.shape), flush=True)
    o, st = _chunk(inp)
    d = inp.to(DEV)
    o_r, st_r = fused_recurrent_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                                 output_final_state=True, cu_seqlens=d.cu_seqlens,
                                                 cu_seqlens_cpu=inp.cu_seqlens)
    torch.cuda.synchronize()
    assert_output_close(o, o_r.float())
    assert_state_close(st, st_r)


def test_varlen_generator_sums_exactly():
    cu = varlen_cu_seqlens(8, 32768, 512, 8192, 1003)
    assert cu[0] == 0 and cu[-1] == 32768 and (cu[1:] > cu[:-1]).all()


def test_chunk_extreme_inputs_stay_finite():
    # x100 inputs (reference test_gdn.py:60-71): large |g| drives exp(gam) to 0; nothing may be NaN
    inp = gdn_inputs(1, 130, 2, 64, dtype=torch.bfloat16, seed=5, h0=True)
    inp.g = inp.g * 100
    inp.v = (inp.v.float() * 100).to(torch.bfloat16)
    o, st = _chunk(inp)
    assert torch.isfinite(o).all() and torch.isfinite(st).all()
    o_ref, st_ref = _oracle(inp)
    assert_output_close(o.cpu(), o_ref, tol=2e-2 * float(o_ref.abs().max()))
    assert_state_close(st.cpu(), st_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_chunk_config0_full_precision_inputs(dtype):
    """BASELINE config 0 (B=1, T=256, H=4, d=64, fp32) through ``chunk_gated_delta_rule``: fp32/fp16
    q/k/v run the token-by-token fp32 kernel, compared with the oracle at the fp32/fp16 bar."""
    print(f"chunk config0 {dtype}", flush=True)
    inp = config_inputs(0)
    inp.q, inp.k, inp.v = inp.q.to(dtype), inp.k.to(dtype), inp.v.to(dtype)
    o, st = _chunk(inp)
    assert o.dtype == dtype
    o_ref, st_ref = _oracle(inp)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)



@pytest.mark.parametrize("case", ["T700_h0", "T640_gva2x", "varlen", "short"])
def test_cooperative_prefill_matches_oracle(case, monkeypatch):
    """The cooperative single-launch prefill (``SORERNN_PREFILL=coop``, K = V = 128 inference): more
    chunks than the ring has slots (the slots are reused), grouped value heads, varlen documents that
    end inside a chunk, and a sequence shorter than a chunk."""
    monkeypatch.setenv("SORERNN_PREFILL", "coop")
    print(f"cooperative prefill {case}", flush=True)
    if case == "T700_h0":
        inp = gdn_inputs(2, 700, 2, 128, dtype=torch.bfloat16, seed=21, h0=True)
    elif case == "T640_gva2x":
        inp = gdn_inputs(1, 640, 2, 128, HV=4, dtype=torch.bfloat16, seed=22, h0=False)
    elif case == "varlen":
        cu = torch.tensor([0, 5, 600, 601, 1000], dtype=torch.long)
        inp = gdn_inputs(1, 1000, 2, 128, HV=2, dtype=torch.bfloat16, seed=23, h0=True, cu_seqlens=cu)
    else:
        inp = gdn_inputs(3, 37, 2, 128, dtype=torch.bfloat16, seed=24, h0=True)
    o, st = _chunk(inp)
    o_ref, st_ref = _oracle(inp)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)
