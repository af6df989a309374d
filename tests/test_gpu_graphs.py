"""GPU: the kernels inside captured HIP graphs (torch.cuda.CUDAGraph) give the eager results on every replay.

A serving loop replays one captured decode step per token, and a training step may capture the
varlen prefill; the fused-norm call clears its progress words with a fill kernel that the graph
holds. The chunk kernel's grid depends only on the number of sequences (not on their
lengths), so a graph captured for one ``cu_seqlens`` stays valid when the lengths change: the
failure documented for FLA's varlen kernels in the reference (``docs/perf/cuda-graphs.md:79-91``,
grid frozen at capture) cannot happen. Each test replays several times with eager work and
synchronisations in between and checks every replay.
"""
import pytest
import torch

from sorernn_amd import chunk_gated_delta_rule, gated_delta_decode_step
from sorernn_amd.synthetic import decode_inputs, gdn_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def test_decode_step_graph_replays_match_eager():
    di = decode_inputs(B=8, H=4, HV=4, D=128, seed=7)
    dev = lambda x: x.to(DEV)  # noqa: E731
    x, cw, g, b = dev(di.x_qkv), dev(di.conv_weight), dev(di.g), dev(di.beta)
    conv_g, st_g = dev(di.conv_state), dev(di.state)
    out_g = torch.empty(8, 1, 4, 128, device=DEV, dtype=x.dtype)
    graph = _capture(lambda: gated_delta_decode_step(x, conv_g, cw, g, b, st_g, 4, 4, 128, out=out_g))
    # reference: the same steps run eagerly from the state the capture left behind
    conv_e, st_e = conv_g.clone(), st_g.clone()
    gen = torch.Generator().manual_seed(3)
    for rep in range(4):
        x.copy_(torch.randn(di.x_qkv.shape, generator=gen).to(x.dtype))  # new token in place
        graph.replay()
        o_e = gated_delta_decode_step(x, conv_e, cw, g, b, st_e, 4, 4, 128)
        torch.cuda.synchronize()
        assert torch.equal(out_g, o_e), f"replay {rep}: output differs"
        assert torch.equal(st_g, st_e), f"replay {rep}: state differs"
        assert torch.equal(conv_g, conv_e), f"replay {rep}: conv cache differs"
        _ = (st_e * 2).sum().item()  # unrelated eager work between replays


def test_varlen_prefill_graph_survives_new_lengths():
    t = 300
    inp = gdn_inputs(1, t, 2, 128, dtype=torch.bfloat16, seed=9, h0=True, cu_seqlens=torch.tensor([0, 10, 100, 300]))
    d = inp.to(DEV)
    cu = d.cu_seqlens.clone()
    o_buf = {}

    def run():
        o, st = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                       output_final_state=True, cu_seqlens=cu, cu_seqlens_cpu=inp.cu_seqlens)
        o_buf["o"], o_buf["st"] = o, st

    graph = _capture(run)
    for rep, bounds in enumerate([[0, 10, 100, 300], [0, 150, 151, 300], [0, 1, 2, 300], [0, 10, 100, 300]]):
        host = torch.tensor(bounds)
        cu.copy_(host.to(DEV))  # same N, new lengths: no re-capture
        graph.replay()
        o_e, st_e = chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, initial_state=d.h0,
                                           output_final_state=True, cu_seqlens=cu, cu_seqlens_cpu=host)
        torch.cuda.synchronize()
        assert torch.equal(o_buf["o"], o_e), f"replay {rep}: output differs for {bounds}"
        assert torch.equal(o_buf["st"], st_e), f"replay {rep}: final state differs for {bounds}"


def test_fused_norm_graph_replays_match_eager():
    """chunk_gated_delta_rule_gated_norm on its epilogue route (8 chains, so epilogue workgroups on
    the free CUs): the progress words are cleared by a fill kernel inside the graph, so every replay,
    with new q, v and gate written in place between replays, equals the eager call bit for bit."""
    from sorernn_amd.ops import chunk_gated_delta_rule_gated_norm

    inp = gdn_inputs(2, 512, 4, 128, dtype=torch.bfloat16, seed=11, h0=True)
    d = inp.to(DEV)
    gen = torch.Generator().manual_seed(12)
    gate = torch.randn(d.v.shape, generator=gen).to(torch.bfloat16).to(DEV)
    w = (1.0 + 0.1 * torch.randn(128, generator=gen)).to(DEV)
    buf = {}

    def run():
        buf["y"], buf["st"] = chunk_gated_delta_rule_gated_norm(d.q, d.k, d.v, d.g, d.beta, gate, w, 1e-6,
                                                                scale=inp.scale, initial_state=d.h0,
                                                                output_final_state=True)

    graph = _capture(run)
    for rep in range(4):
        d.q.copy_(torch.randn(d.q.shape, generator=gen).to(torch.bfloat16))
        d.v.copy_(torch.randn(d.v.shape, generator=gen).to(torch.bfloat16))
        gate.copy_(torch.randn(gate.shape, generator=gen).to(torch.bfloat16))
        graph.replay()
        y_e, st_e = chunk_gated_delta_rule_gated_norm(d.q, d.k, d.v, d.g, d.beta, gate, w, 1e-6, scale=inp.scale,
                                                      initial_state=d.h0, output_final_state=True)
        torch.cuda.synchronize()
        assert torch.equal(buf["y"], y_e), f"replay {rep}: output differs"
        assert torch.equal(buf["st"], st_e), f"replay {rep}: final state differs"
        _ = (st_e * 2).sum().item()  # unrelated eager work between replays
