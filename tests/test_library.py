"""torch.library registration (CPU): the ops trace as single graph nodes with fake tensors.

The reference's per-Block ``torch.compile`` breaks its graph at FLA's autograd function
(``RUNBOOK_4090.md:203-208``). Here the GDN operators are custom ops with fake implementations and
registered autograd formulas, so a trace of the layer's forward and backward with fake CUDA tensors
(no GPU needed: nothing runs) records them as ``sorernn::*`` nodes. The Python size formulas used
by the fake implementations must equal the library's size functions.
"""
import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

from sorernn_amd import _lib, library
from sorernn_amd.gdn_layer import GatedDeltaNet, GDNLayerConfig


@pytest.mark.parametrize("prefill", [None, "coop"])
def test_size_formulas_match_the_library(prefill, monkeypatch):
    """Both with the default two-kernel prefill and with the cooperative prefill selected, whose ring
    the forward workspace covers only then."""
    if prefill is None:
        monkeypatch.delenv("SORERNN_PREFILL", raising=False)
    else:
        monkeypatch.setenv("SORERNN_PREFILL", prefill)
    lib = _lib.load()
    for (b, t, hv, kd, vd, n, varlen) in [(4, 4096, 16, 128, 128, 4, False), (1, 100, 3, 64, 64, 5, True),
                                          (2, 65, 2, 128, 64, 2, False), (1, 32768, 16, 128, 128, 8, True),
                                          (1, 100, 3, 128, 128, 300, True)]:
        assert library.states_bytes(b, t, hv, kd, vd, n, varlen) == lib.gdn_chunk_states_size(b, t, hv, kd, vd, n, int(varlen))
        assert library.fwd_workspace_bytes(b, t, hv, n, varlen) == lib.gdn_chunk_workspace_size(b, t, hv, n, int(varlen))
        assert library.bwd_workspace_bytes(b, t, hv, kd, vd, n, varlen) == lib.gdn_chunk_bwd_workspace_size(
            b, t, hv, kd, vd, n, int(varlen))


def _trace_layer_forward(kernel_gate):
    torch.manual_seed(0)
    cfg = GDNLayerConfig(d_model=128, gdn_qk_heads=2, gdn_v_heads=4, gdn_head_dim=64, gdn_kernel_gate=kernel_gate,
                         gdn_fla_conv=True, fused_norm_gate=True)
    layer = GatedDeltaNet(cfg).to(torch.bfloat16)
    params = dict(layer.named_parameters())

    def fwd(x, *ps):
        return torch.func.functional_call(layer, dict(zip(params, ps)), (x,))

    # fake CUDA tensors: the ops check the device, nothing executes (the backward is not traced here:
    # the autograd engine needs a device; the GPU tests run it, also under torch.compile)
    with torch._subclasses.fake_tensor.FakeTensorMode() as mode:
        xf = mode.from_tensor(torch.empty(2, 96, 128, dtype=torch.bfloat16, device="meta")).to("cuda").requires_grad_(True)
        pf = [mode.from_tensor(torch.empty(p.shape, dtype=p.dtype, device="meta")).to("cuda").requires_grad_(True)
              for p in params.values()]
    g = make_fx(fwd, tracing_mode="fake")(xf, *pf)
    return [str(n.target) for n in g.graph.nodes if n.op == "call_function"]


def test_layer_forward_traces_into_custom_ops():
    for kernel_gate in (True, False):
        names = " ".join(_trace_layer_forward(kernel_gate))
        assert names.count("sorernn.causal_conv1d_fwd") == 3, names
        assert names.count("sorernn.chunk_gated_delta_rule_fwd") == 1, names
        assert names.count("sorernn.rms_norm_gated_fwd") == 1, names


def test_backward_formulas_are_registered():
    for op in ("chunk_gated_delta_rule_fwd", "causal_conv1d_fwd", "l2norm_fwd", "rms_norm_gated_fwd"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"sorernn::{op}", "Autograd"), op
    # the backward ops' fake implementations give the gradient shapes (and the empty placeholders)
    with torch._subclasses.fake_tensor.FakeTensorMode() as mode:
        mk = lambda *shape, dt=torch.bfloat16: mode.from_tensor(torch.empty(*shape, dtype=dt, device="meta")).to("cuda")  # noqa: E731
        q, k, v = mk(1, 130, 2, 64), mk(1, 130, 2, 64), mk(1, 130, 4, 64)
        g, beta, do = mk(1, 130, 4, dt=torch.float32), mk(1, 130, 4, dt=torch.float32), mk(1, 130, 4, 64)
        states = mk(library.states_bytes(1, 130, 4, 64, 64, 1, False), dt=torch.uint8)
        ws = mk(library.fwd_workspace_bytes(1, 130, 4, 1, False), dt=torch.uint8)
        out = library.chunk_bwd(q, k, v, g, beta, do, None, states, ws, None, None, None, 0.125, 0, 1, True)
        assert [tuple(x.shape) for x in out] == [(1, 130, 2, 64), (1, 130, 2, 64), (1, 130, 4, 64), (1, 130, 4),
                                                 (1, 130, 4), (1, 4, 64, 64), (0,), (0,)]


def test_eager_fast_path_yields_to_tracing_and_dispatch_modes():
    """Plain eager inference calls the op implementation directly; anything that records, traces or
    fakes tensors must see the registered torch.library op instead."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.utils._python_dispatch import TorchDispatchMode

    from sorernn_amd.ops import _plain_eager

    x = torch.zeros(2)
    assert _plain_eager(x)

    class Record(TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    with Record():
        assert not _plain_eager(x)
    with FakeTensorMode() as mode:
        assert not _plain_eager(mode.from_tensor(x))
    assert not torch.compile(lambda t: torch.tensor(_plain_eager(t)), fullgraph=True, backend="eager")(x)
