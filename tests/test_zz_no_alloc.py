"""``gdn_chunk_fwd_noalloc`` (the allocation-free prefill entry point) against ``gdn_chunk_fwd``.

Both run the same two kernels; only the workspace differs (the library's built-in scratch array vs a
caller buffer), so outputs and final states must agree bit for bit. Two calls in a row, the second
with a smaller input (the array keeps the first call's contents), then varlen calls (one of many
documents without states, which takes the persistent state grid), all through the C ABI. Oversized inputs are rejected on the host before any launch.
"""
import pytest
import torch

from sorernn_amd import _lib
from sorernn_amd.synthetic import gdn_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(entry, inp, flags=0, final_state=True):
    d = inp.to(DEV)
    b, t, h, kd = d.q.shape
    hv, vd = d.v.shape[2], d.v.shape[3]
    n = b if d.cu_seqlens is None else d.cu_seqlens.numel() - 1
    o = torch.empty_like(d.v)
    final = torch.empty(n, hv, kd, vd, device=DEV, dtype=torch.float32) if final_state else None
    args = [_lib.ptr(d.q), _lib.ptr(d.k), _lib.ptr(d.v), _lib.ptr(d.g), _lib.ptr(d.beta), _lib.ptr(d.h0),
            _lib.ptr(o), _lib.ptr(final), _lib.ptr(d.cu_seqlens), b, t, h, hv, kd, vd, n,
            _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32, inp.scale, flags, None, None]
    if entry == "gdn_chunk_fwd":
        nbytes = int(_lib.load().gdn_chunk_workspace_size(b, t, hv, n, int(d.cu_seqlens is not None)))
        ws = torch.full((max(nbytes, 1),), 0x7F, dtype=torch.uint8, device=DEV)
        args += [_lib.ptr(ws), nbytes]
    _lib.call(entry, *args, _lib.stream_of(o))
    torch.cuda.synchronize()
    return o.cpu(), None if final is None else final.cpu()


def _same(inp, final_state=True):
    o1, s1 = _run("gdn_chunk_fwd", inp, final_state=final_state)
    o2, s2 = _run("gdn_chunk_fwd_noalloc", inp, final_state=final_state)
    assert torch.equal(o1, o2), "outputs differ"
    if final_state:
        assert torch.equal(s1, s2), "final states differ"


def test_noalloc_matches_workspace_entry_twice_then_smaller():
    print("noalloc: config-1 shape, then a smaller call", flush=True)
    _same(gdn_inputs(4, 4096, 16, 128, dtype=torch.bfloat16, seed=1001, h0=True))
    _same(gdn_inputs(2, 300, 4, 64, V=128, HV=8, dtype=torch.bfloat16, seed=5, h0=True))


def test_noalloc_matches_workspace_entry_varlen():
    print("noalloc: varlen", flush=True)
    cu = torch.tensor([0, 1, 70, 200, 777, 1024])
    _same(gdn_inputs(1, 1024, 2, 128, HV=4, dtype=torch.bfloat16, seed=9, h0=True, cu_seqlens=cu))


def test_noalloc_matches_workspace_entry_persistent_grid(monkeypatch):
    """Many documents, no initial or final state: both entries run the persistent state grid (the
    index kernel's order and chunk map in the scratch array); then the varlen call with states again.
    1,000 documents of 1-100 tokens at HV = 8 (8,000 chains, ~400k token-heads): the default
    prefill's workspace fits the built-in array, where the cooperative prefill's ring (counted only
    when SORERNN_PREFILL=coop selects it) would not."""
    print("noalloc: persistent grid", flush=True)
    monkeypatch.delenv("SORERNN_PREFILL", raising=False)
    gen = torch.Generator().manual_seed(12)
    lens = torch.randint(1, 101, (1000,), generator=gen).tolist()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist())
    lib = _lib.load()
    need = int(lib.gdn_chunk_workspace_size(1, int(cu[-1]), 8, 1000, 1))
    assert need <= int(lib.gdn_chunk_fwd_noalloc_max_workspace()), need
    _same(gdn_inputs(1, int(cu[-1]), 2, 128, HV=8, dtype=torch.bfloat16, seed=13, cu_seqlens=cu), final_state=False)
    cu2 = torch.tensor([0, 1, 70, 200, 777, 1024])
    _same(gdn_inputs(1, 1024, 2, 128, HV=4, dtype=torch.bfloat16, seed=9, h0=True, cu_seqlens=cu2))


def test_noalloc_rejects_sizes_beyond_its_array():
    cap = int(_lib.load().gdn_chunk_fwd_noalloc_max_workspace())
    tokens = cap // (16 * 128) + 64  # more token-heads than the array holds at HV = 16
    # null tensor pointers: the size check fails first; were it ever skipped, the entry point's
    # null-pointer check would still stop the call on the host before any launch
    with pytest.raises(ValueError, match="scratch array"):
        _lib.call("gdn_chunk_fwd_noalloc", None, None, None, None, None, None, None, None, None, 1, tokens, 16, 16,
                  128, 128, 1, _lib.DTYPE_BF16, _lib.DTYPE_F32, _lib.DTYPE_F32, 0.088, 0, None, None, None)
