"""GPU: the varlen index work of the chunked prefill, bit-exact.

With ``cu_seqlens`` the prefill's first launch, ``gated_delta_chunk_index_kernel``, writes into the
caller's workspace (after the T - I rows, 256-byte aligned):
  chunk_first[N + 1]  int32: chunks before each sequence, sum of ceil(L / 64) (the prep kernel's
                      chunk -> sequence map; reference: ``chunk_indices_without_sync``,
                      sore/model/gdn.py:31-51, n_chunks = sum ceil(L_i / C) from cu_seqlens_cpu);
  order[N]            int32: sequences by chunk count, longest first, ties by index, for N <= 2048
                      (a bitonic sort in LDS); the identity above that.
Both are read back through the C ABI and compared with a host computation, at N = 1, 7, 1025 (the
block scan's second tile), 2048, 2049 and 5000 (identity order), with int32 and int64 cu_seqlens;
the chunk outputs at N > 2048 are compared with the oracle on a few documents. Integer work: exact.
"""
import numpy as np
import pytest
import torch

from oracle import recurrent_gated_delta_rule
from sorernn_amd import _lib, chunk_gated_delta_rule
from sorernn_amd.synthetic import gdn_inputs
from tests.parity import assert_output_close, assert_state_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
C = 64


def _lengths(n, seed):
    rng = np.random.default_rng(seed)
    # mostly short documents, some spanning several chunks, so chunk counts tie and differ
    lens = rng.choice([1, 2, 3, 63, 64, 65, 130, 200], size=n)
    return lens.astype(np.int64)


def _host_index(lens):
    nch = -(-lens // C)
    first = np.concatenate([[0], np.cumsum(nch)]).astype(np.int32)
    if len(lens) > 2048:
        order = np.arange(len(lens), dtype=np.int32)
    else:
        order = np.array(sorted(range(len(lens)), key=lambda i: (-int(nch[i]), i)), dtype=np.int32)
    return first, order


def _run_index(lens, cu_dtype, hv=1, kd=64):
    t = int(lens.sum())
    n = len(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=cu_dtype)
    inp = gdn_inputs(1, t, 1, kd, HV=hv, dtype=torch.bfloat16, seed=11, h0=True, cu_seqlens=cu.long())
    d = inp.to(DEV)
    cud = cu.to(DEV)
    o = torch.empty_like(d.v)
    fin = torch.empty(n, hv, kd, kd, device=DEV)
    lib = _lib.load()
    nbytes = int(lib.gdn_chunk_workspace_size(1, t, hv, n, 1))
    ws = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=DEV)
    flags = _lib.FLAG_CU_INT32 if cu_dtype == torch.int32 else 0
    _lib.call("gdn_chunk_fwd", d.q.data_ptr(), d.k.data_ptr(), d.v.data_ptr(), d.g.data_ptr(), d.beta.data_ptr(),
              d.h0.data_ptr(), o.data_ptr(), fin.data_ptr(), cud.data_ptr(), 1, t, 1, hv, kd, kd, n,
              _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32, inp.scale, flags, None, None, ws.data_ptr(), nbytes,
              _lib.stream_of(o))
    torch.cuda.synchronize()
    align = lambda b: (b + 255) // 256 * 256  # noqa: E731
    t_bytes = align(t * hv * C * 2)
    raw = ws.cpu().numpy()
    first = raw[t_bytes:t_bytes + 4 * (n + 1)].view(np.int32)
    o_off = t_bytes + align(4 * (n + 1))
    order = raw[o_off:o_off + 4 * n].view(np.int32)
    return first, order, inp, o.cpu(), fin.cpu()


@pytest.mark.parametrize("n", [1, 7, 1025, 2048, 2049, 5000])
@pytest.mark.parametrize("cu_dtype", [torch.int64, torch.int32], ids=["i64", "i32"])
def test_index_kernel_bit_exact(n, cu_dtype):
    print(f"index kernel N={n} {cu_dtype}", flush=True)
    lens = _lengths(n, seed=n)
    first, order, *_ = _run_index(lens, cu_dtype)
    h_first, h_order = _host_index(lens)
    assert np.array_equal(first, h_first), "chunk_first differs from the host scan"
    assert np.array_equal(order, h_order), "order differs from the host sort"


def test_many_documents_match_oracle():
    """N = 2049 > 2048 (identity order, two scan tiles): documents at both ends, a multi-chunk one
    and single-token ones against the oracle from their own initial states."""
    lens = _lengths(2049, seed=3)
    first, order, inp, o, fin = _run_index(lens, torch.int64)
    cu = np.concatenate([[0], np.cumsum(lens)])
    picks = [0, 1, int(np.argmax(lens)), 1024, 2047, 2048]
    for n in picks:
        a, e = int(cu[n]), int(cu[n + 1])
        o_ref, st_ref = recurrent_gated_delta_rule(inp.q[:, a:e], inp.k[:, a:e], inp.v[:, a:e], inp.g[:, a:e],
                                                   inp.beta[:, a:e], inp.scale, inp.h0[n:n + 1], True)
        assert_output_close(o[:, a:e], o_ref, what=f"o of document {n} (length {e - a})")
        assert_state_close(fin[n:n + 1], st_ref, what=f"final state of document {n}")


def test_op_cu_seqlens_cpu_is_exact():
    """The op with and without cu_seqlens_cpu: same values, same kernels, bitwise equal outputs and
    final states (reference tests/model/test_lm.py:339-361)."""
    lens = np.array([1, 3, 70, 200, 64, 65, 130, 1])
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]))
    inp = gdn_inputs(1, int(lens.sum()), 2, 128, HV=4, dtype=torch.bfloat16, seed=12, h0=True, cu_seqlens=cu)
    d = inp.to(DEV)
    runs = []
    for cpu in (None, None, cu):
        o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                       output_final_state=True, cu_seqlens=d.cu_seqlens, cu_seqlens_cpu=cpu)
        runs.append((o.cpu(), st.cpu()))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1]), "two identical runs differ"
    assert torch.equal(runs[2][0], runs[0][0]) and torch.equal(runs[2][1], runs[0][1])
