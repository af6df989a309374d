"""GPU parity of the chunked rule's backward (``chunk_gated_delta_rule`` under autograd).

The reference trains through FLA's autograd function and checks FLA's gradients against autograd
through its torch recurrence (tests/model/test_gdn.py:94-101,156-162). Here the HIP backward is
compared with the fp64 oracle backward ``chunk_gated_delta_rule_bwd_ref`` (itself pinned against
autograd through the token recurrence in tests/test_oracle.py) on the same bf16 inputs and
cotangents, with the reference's tolerance (``tests/parity.py::assert_grad_close``). The kernel
options (in-kernel L2 norm, gate, beta sigmoid) are checked against autograd through the oracle's
composition of those functions.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import chunk_gated_delta_rule_bwd_ref, recurrent_gated_delta_rule
from sorernn_amd import chunk_gated_delta_rule
from sorernn_amd.synthetic import config_inputs, gdn_inputs
from tests.parity import assert_grad_close, assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cotangents(inp, seed, n):
    gen = torch.Generator().manual_seed(seed)
    b, t, hv, vd = inp.v.shape
    kd = inp.q.shape[-1]
    do = torch.randn(b, t, hv, vd, generator=gen).to(torch.bfloat16)
    dht = torch.randn(n, hv, kd, vd, generator=gen) * 0.1
    return do, dht


def _gpu_grads(inp, do, dht, with_h0=True):
    leaves = [x.to(DEV).requires_grad_(True) for x in (inp.q, inp.k, inp.v, inp.g, inp.beta)]
    h0 = inp.h0.to(DEV).requires_grad_(True) if (with_h0 and inp.h0 is not None) else None
    cu = None if inp.cu_seqlens is None else inp.cu_seqlens.to(DEV)
    o, st = chunk_gated_delta_rule(*leaves, scale=inp.scale, initial_state=h0, output_final_state=True,
                                   cu_seqlens=cu, cu_seqlens_cpu=inp.cu_seqlens)
    torch.autograd.backward([o, st], [do.to(DEV), dht.to(DEV)])
    torch.cuda.synchronize()
    grads = [x.grad for x in leaves] + [None if h0 is None else h0.grad]
    return o.detach(), st.detach(), grads


def _check(inp, do, dht, grads):
    cu = None if inp.cu_seqlens is None else inp.cu_seqlens.long()
    ref = chunk_gated_delta_rule_bwd_ref(inp.q, inp.k, inp.v, inp.g, inp.beta, do, inp.scale, inp.h0, dht, cu_seqlens=cu)
    for name, out, r in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), grads, ref):
        if out is None:
            continue
        rel = assert_grad_close(out, r, name)
        print(f"  {name}: max err / max|ref| = {rel:.2e}", flush=True)


@pytest.mark.parametrize("t", [256, 200, 64, 1], ids=lambda t: f"T{t}")
def test_chunk_bwd_small_matches_oracle(t):
    print(f"chunk bwd T={t}", flush=True)
    inp = gdn_inputs(2, t, 2, 64, dtype=torch.bfloat16, seed=2000 + t, h0=True)
    do, dht = _cotangents(inp, 3000 + t, 2)
    o, st, grads = _gpu_grads(inp, do, dht)
    o_ref, st_ref = recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
    assert_output_close(o.cpu(), o_ref)
    assert_state_close(st.cpu(), st_ref)
    _check(inp, do, dht, grads)


@pytest.mark.parametrize("kv", [(128, 128), (64, 64), (128, 64), (64, 128)], ids=lambda x: f"K{x[0]}V{x[1]}")
def test_chunk_bwd_head_dims(kv):
    kd, vd = kv
    print(f"chunk bwd K={kd} V={vd}", flush=True)
    inp = gdn_inputs(2, 300, 3, kd, V=vd, dtype=torch.bfloat16, seed=41, h0=True)
    do, dht = _cotangents(inp, 42, 2)
    _, _, grads = _gpu_grads(inp, do, dht)
    _check(inp, do, dht, grads)


@pytest.mark.parametrize("cu", [[0, 1, 3, 4, 70, 200, 512], [0, 63, 64, 65, 129, 300]], ids=["short_docs", "chunk_edges"])
@pytest.mark.parametrize("rep", [1, 2], ids=["no_gva", "gva2x"])
def test_chunk_bwd_varlen_gva_matches_oracle(cu, rep):
    print(f"chunk bwd varlen cu={cu} rep={rep}", flush=True)
    cu_t = torch.tensor(cu, dtype=torch.long)
    inp = gdn_inputs(1, cu[-1], 2, 128, HV=2 * rep, dtype=torch.bfloat16, seed=5, h0=True, cu_seqlens=cu_t)
    do, dht = _cotangents(inp, 6, len(cu) - 1)
    _, _, grads = _gpu_grads(inp, do, dht)
    _check(inp, do, dht, grads)


def test_chunk_bwd_without_initial_state_or_final_grad():
    inp = gdn_inputs(1, 130, 2, 128, dtype=torch.bfloat16, seed=8, h0=False)
    gen = torch.Generator().manual_seed(9)
    do = torch.randn(inp.v.shape, generator=gen).to(torch.bfloat16)
    leaves = [x.to(DEV).requires_grad_(True) for x in (inp.q, inp.k, inp.v, inp.g, inp.beta)]
    o, st = chunk_gated_delta_rule(*leaves, scale=inp.scale)
    assert st is None
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    ref = chunk_gated_delta_rule_bwd_ref(inp.q, inp.k, inp.v, inp.g, inp.beta, do, inp.scale)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), leaves, ref):
        assert_grad_close(x.grad, r, name)


def test_chunk_bwd_kernel_options_match_autograd():
    # raw inputs as sore/model/gdn.py passes them with gdn_kernel_gate: unnormalised q/k, a, b logits
    gen = torch.Generator().manual_seed(31)
    t, h, hv, d = 200, 2, 4, 128
    q = (torch.randn(1, t, h, d, generator=gen) * 2).to(torch.bfloat16)
    k = (torch.randn(1, t, h, d, generator=gen) * 2).to(torch.bfloat16)
    v = torch.randn(1, t, hv, d, generator=gen).to(torch.bfloat16)
    a = torch.randn(1, t, hv, generator=gen)
    b = torch.randn(1, t, hv, generator=gen)
    A_log = torch.empty(hv).uniform_(1, 16, generator=gen).log()
    dt_bias = torch.randn(hv, generator=gen) * 0.3
    do = torch.randn(1, t, hv, d, generator=gen).to(torch.bfloat16)
    cu = torch.tensor([0, 5, 77, 200])
    leaves = [x.to(DEV).requires_grad_(True) for x in (q, k, v, a, b, A_log, dt_bias)]
    o, _ = chunk_gated_delta_rule(*leaves[:5], initial_state=None, use_qk_l2norm_in_kernel=True,
                                  use_beta_sigmoid_in_kernel=True, use_gate_in_kernel=True, A_log=leaves[5],
                                  dt_bias=leaves[6], cu_seqlens=cu.to(DEV), cu_seqlens_cpu=cu)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    # autograd through the oracle composition, fp64
    ref_leaves = [x.double().requires_grad_(True) for x in (q, k, v, a, b, A_log, dt_bias)]
    qr, kr, vr, ar, br, alr, dtr = ref_leaves
    g_ref = -alr.exp() * F.softplus(ar + dtr)
    beta_ref = br.sigmoid()
    o_ref, _ = recurrent_gated_delta_rule(F.normalize(qr, dim=-1), F.normalize(kr, dim=-1), vr, g_ref, beta_ref,
                                          d**-0.5, None, False, cu_seqlens=cu)
    o_ref.backward(do.double())
    assert_output_close(o.cpu(), o_ref.detach())
    for name, x, r in zip(("dq", "dk", "dv", "da", "db_logit", "dA_log", "ddt_bias"), leaves, ref_leaves):
        frac = 5e-2 if name in ("dA_log", "ddt_bias") else 5e-3
        rel = assert_grad_close(x.grad, r.grad, name, atol_frac=frac)
        print(f"  {name}: max err / max|ref| = {rel:.2e}", flush=True)


def test_chunk_bwd_config1_slice_matches_oracle():
    # full config-1 backward on the GPU; the oracle on batch row 2, heads 3 and 12 (chains are independent)
    inp = config_inputs(1)
    print("chunk bwd config1", flush=True)
    do, dht = _cotangents(inp, 77, 4)
    _, _, grads = _gpu_grads(inp, do, dht)
    sl = lambda x: x[2:3, :, [3, 12]]  # noqa: E731
    ref = chunk_gated_delta_rule_bwd_ref(sl(inp.q), sl(inp.k), sl(inp.v), sl(inp.g), sl(inp.beta), sl(do), inp.scale,
                                         inp.h0[2:3, [3, 12]], dht[2:3, [3, 12]])
    for name, out, r in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), grads, ref):
        out = out[2:3, [3, 12]] if name == "dh0" else sl(out)
        rel = assert_grad_close(out, r, name)
        print(f"  {name}: max err / max|ref| = {rel:.2e}", flush=True)


def test_chunk_bwd_is_linear_in_the_cotangents():
    inp = gdn_inputs(1, 256, 2, 128, dtype=torch.bfloat16, seed=12, h0=True)
    do, dht = _cotangents(inp, 13, 1)
    _, _, g1 = _gpu_grads(inp, do, dht)
    _, _, g2 = _gpu_grads(inp, (do.float() * 4).to(torch.bfloat16), dht * 4)
    # exact up to the order of the per-token LDS sums (dg, dbeta)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), g1, g2):
        err = float((b.double() - 4 * a.double()).abs().max())
        assert err <= 1e-5 * float((4 * a.double()).abs().max()), f"{name}: {err:.3e}"
