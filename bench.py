#!/usr/bin/env python3
"""Benchmark of the GDN token-mixing path on one MI355X (BASELINE.json metric).

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line. A step is one
``chunk_gated_delta_rule`` call over BASELINE config 1 (B=4, T=4096, H=16, d_k=d_v=128, bf16 q/k/v,
fp32 g/beta/h0, final state out), inputs already resident in HBM; ``value`` is prefill tokens/s, from
launches alternating over two input sets (2 x 281 MB, more than the 256 MB Infinity Cache), so every
launch reads its inputs from DRAM; the one-input-set (cache-resident) rate is reported beside it.
Every workload first runs its own step untimed for 100 ms (``settle``: from idle the GPU's clocks
need ~35 ms of this load to reach their sustained rate), then W warmup steps, then the K timed steps;
``cold_ms_per_step`` / ``cold_value`` report the prefill's first K steps after W warmup steps
without that phase.

The same line carries
- ``roofline``: the chunked prefill op -- its two kernels, gated_delta_chunk_prep_kernel (the
  per-chunk (I + A)^-1) then gated_delta_chunk_kernel (the state recurrence), launched back to back
  on one stream -- against bf16 dense MFMA peak, from HIP events around each op launch on that
  stream; algorithmic FLOPs per launch = (10 C^2 d + 6 C d^2) per (chunk, head) x 4096 chunk-heads
  = 47,244,640,256 (C = 64, d = 128, solve excluded); ``traffic`` (HBM bytes per launch, both
  kernels) comes from the committed rocprofv3 PMC summary when present;
- ``decode``: config 2, 1000 back-to-back fused decode steps (conv cache + SiLU + L2 norm + state
  update, state updated in place) with HBM bytes/step = 141,664,256. The headline steps rotate over
  5 state/conv copies (5 x 73 MB > the 256 MB Infinity Cache), so every step reads its state from
  DRAM, as the layers of a model do; the cache-resident rate (one state) is reported beside it;
- ``varlen``: config 3 (8 packed documents, 32768 tokens);
- ``varlen_docs``: the reference model's call (zero initial state, no final state) on its real
  document-length distribution: 8 windows of 4096 tokens filled from the reference's corpus sample
  (``tests/golden/doc_lengths_pt.json``, drawn as the reference's bench ``--doc-lengths`` does);
- ``train``: config 1 under autograd -- the training forward (which also saves the bf16 state
  entering every chunk) and the backward (dq, dk, dv, dg, dbeta, dh0), timed separately with HIP
  events; backward algorithmic FLOPs = (22 C^2 d + 14 C d^2) per (chunk, head);
- ``block_pair``: config 4 -- the GDN layer and the gated attention layer (B=2, T=8192, hidden 2048)
  forward, each timed whole, plus the flash-attention kernel alone against bf16 peak (causal FLOPs
  4 d T (T + 1) / 2 per head and batch row);
- ``cpu_baseline``: the CPU oracle (``oracle/``, torch fp32 recurrence) on the GPU box's host
  cores over the full config-1 input, config 3's per-document loop over its full input, plus 100
  decode steps of config 2.

Each GPU workload runs in its own child process (``bench.py --part NAME`` prints its raw
measurements as JSON), so every workload is measured in a fresh HIP context and allocator, as it would
run alone; this process never initialises the GPU and runs the CPU baseline itself. A failing
workload ends the bench with its status. ``--only NAME`` runs one workload for profiler runs.
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
C = 64
PREFILL_KERNELS = ("gated_delta_chunk_prep_kernel", "gated_delta_chunk_kernel")  # one op = these two launches


def chunk_flops(lengths, heads: int, d: int) -> int:
    """Algorithmic forward FLOPs: sum over chunks of (10 c^2 d + 6 c d^2) x heads, c = real chunk length."""
    total = 0
    for L in lengths:
        full, rem = divmod(L, C)
        total += full * (10 * C * C * d + 6 * C * d * d)
        if rem:
            total += 10 * rem * rem * d + 6 * rem * d * d
    return total * heads


def chunk_flops_causal(lengths, heads: int, d: int) -> int:
    """The same with the intra-chunk C x C products counted over their causal half only:
    (5 c^2 d + 6 c d^2) x heads per chunk (36.51 GFLOP at config 1)."""
    total = 0
    for L in lengths:
        full, rem = divmod(L, C)
        total += full * (5 * C * C * d + 6 * C * d * d)
        if rem:
            total += 5 * rem * rem * d + 6 * rem * d * d
    return total * heads


def chunk_bwd_flops(lengths, heads: int, d: int) -> int:
    """Algorithmic backward FLOPs: per chunk (c tokens) 22 c^2 d + 14 c d^2 (the recomputed Y and Delta,
    the seven c x d x d products with S or dS' and the eleven c x c x d products), times heads."""
    total = 0
    for L in lengths:
        full, rem = divmod(L, C)
        total += full * (22 * C * C * d + 14 * C * d * d)
        if rem:
            total += 22 * rem * rem * d + 14 * rem * d * d
    return total * heads


def train_step_times(torch, inp, steps: int):
    """(training forward ms, backward ms) of chunk_gated_delta_rule under autograd, HIP events per step.

    The steps run back to back, one synchronisation after the last. The host then runs ahead of
    the GPU, as in a training loop, and each event span is the GPU time of that forward or backward.
    A synchronisation after every step would put the host's launch latency for the next forward
    (the GPU idle until the first kernel arrives) into the forward's span."""
    from sorernn_amd import chunk_gated_delta_rule

    leaves = [x.detach().clone().requires_grad_(True) for x in (inp.q, inp.k, inp.v, inp.g, inp.beta, inp.h0)]
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(inp.v.shape, generator=gen).to(torch.bfloat16).to(inp.q.device)
    dht = (torch.randn(inp.h0.shape, generator=gen) * 0.1).to(inp.q.device)

    def fwd():
        return chunk_gated_delta_rule(*leaves[:5], scale=inp.scale, initial_state=leaves[5], output_final_state=True)

    def bwd(o, st):
        torch.autograd.grad([o, st], leaves, [do, dht])

    for _ in range(2):
        bwd(*fwd())
    settle(torch, lambda: bwd(*fwd()))
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for e in ev:
        e[0].record()
        o, st = fwd()
        e[1].record()
        bwd(o, st)
        e[2].record()
    torch.cuda.synchronize()
    tf = sum(e[0].elapsed_time(e[1]) for e in ev)
    tb = sum(e[1].elapsed_time(e[2]) for e in ev)
    return tf / steps, tb / steps


def decode_bytes(B=64, H=16, HV=16, D=128, W=4) -> int:
    state = B * HV * D * D * 4 * 2  # read + write
    ch = (2 * H + HV) * D
    qkv = B * ch * 2  # pre-conv q|k|v bf16
    out = B * HV * D * 2
    gates = B * HV * 4 * 2
    conv = B * ch * W * 2 * 2 + ch * W * 4  # cache read + write, fp32 weight
    return state + qkv + out + gates + conv


def attn_flops(B: int, T: int, HQ: int, D: int) -> int:
    """Causal attention FLOPs: QK^T and PV over the (T (T + 1) / 2) allowed pairs, 2 x 2 D each, per head."""
    return 4 * D * HQ * B * (T * (T + 1) // 2)


def block_pair(torch, steps: int) -> dict:
    """the GDN layer and the gated attention layer at B=2, T=8192, hidden 2048, bf16,
    random-init weights ~N(0, 0.02); forward of each layer timed with HIP events, plus the attention
    kernel alone (its causal FLOPs against bf16 peak) and the chunked GDN op alone."""
    from sorernn_amd.attention import AttnLayerConfig, GatedAttention, attn_qk_norm_rope, gated_attention
    from sorernn_amd.gdn_layer import GatedDeltaNet, GDNLayerConfig

    B, T, Dm, H, Dh, HKV = 2, 8192, 2048, 16, 128, 4
    torch.manual_seed(1004)
    # the caller flags of the reference's training presets (sore/model/config.py:116,123)
    gdn = GatedDeltaNet(GDNLayerConfig(d_model=Dm, gdn_qk_heads=H, gdn_v_heads=H, gdn_head_dim=Dh, gdn_kernel_gate=True,
                                       gdn_fla_conv=True, fused_norm_gate=True))
    attn = GatedAttention(AttnLayerConfig(d_model=Dm, attn_heads=H, attn_kv_heads=HKV, attn_head_dim=Dh,
                                          rope_theta=1e6, rope_partial=0.25))
    with torch.no_grad():
        for mod in (gdn, attn):
            for name, prm in mod.named_parameters():
                if name.endswith("proj.weight"):
                    prm.normal_(0, 0.02)
    gdn = gdn.to("cuda", torch.bfloat16)
    attn = attn.to("cuda", torch.bfloat16)
    gen = torch.Generator().manual_seed(1004)
    x = torch.randn(B, T, Dm, generator=gen).to(torch.bfloat16).to("cuda")
    out = {"workload": "config4: B=2, T=8192, hidden 2048, bf16 weights ~N(0,0.02); GDN layer (H=16, d=128, "
                       "in-kernel gate) and gated attention layer (16 q / 4 kv heads, d=128, RoPE theta=1e6 on "
                       "25% of dims, sigmoid output gate), forward"}
    with torch.no_grad():
        # gdn_layer: the inference route (fused projections, prologue and norm epilogue);
        # gdn_layer_unfused_epilogue: the same with the chunk op and the norm as two calls;
        # gdn_layer_reference_route:
        # the reference's call expressions (three convs, chunked rule with in-kernel q/k L2 norm),
        # the route the layer takes under autograd
        def unfused_epilogue():  # the chunk op and the norm kernel as two calls (not the layer's default)
            gdn.fused_epilogue = False
            try:
                return gdn(x)
            finally:
                gdn.fused_epilogue = True

        for name, fn in (("gdn_layer", lambda: gdn(x)), ("gdn_layer_reference_route", lambda: gdn._forward_reference(x)),
                         ("gdn_layer_unfused_epilogue", unfused_epilogue), ("attn_layer", lambda: attn(x))):
            for _ in range(2):
                fn()
            settle(torch, fn)
            ms, _ = time_launches(torch, fn, steps)
            out[f"{name}_ms"] = round(ms, 4)
        # the attention kernel alone on the layer's own q, k, v, gate
        proj = torch.nn.functional.linear(x, attn._fused_weight(torch.bfloat16))
        nq, nkv = H * Dh, HKV * Dh
        q, k = attn_qk_norm_rope(proj[..., :nq], proj[..., 2 * nq:2 * nq + nkv], attn.q_norm.weight,
                                 attn.k_norm.weight, H, HKV, attn.rotary.rot_dim, 1e6)
        v, gate = proj[..., 2 * nq + nkv:], proj[..., nq:2 * nq]
        fa = lambda: gated_attention(q, k, v, gate)  # noqa: E731
        fa()
        settle(torch, fa)
        _, fa_ms = time_launches(torch, fa, steps)
        fl = attn_flops(B, T, H, Dh)
        # the layer's GDN call alone at this shape (synthetic config-1 distributions, bf16 gate):
        # the chunked op, the op followed by the norm kernel, and the op with the norm in the call
        from sorernn_amd import chunk_gated_delta_rule, rms_norm_gated
        from sorernn_amd.ops import chunk_gated_delta_rule_gated_norm
        from sorernn_amd.synthetic import gdn_inputs
        gi = gdn_inputs(B, T, H, Dh, dtype=torch.bfloat16, seed=1004).to("cuda")
        og = torch.randn(B, T, H, Dh, device="cuda").to(torch.bfloat16)
        ow = torch.rand(Dh, device="cuda") + 0.5
        op = lambda: chunk_gated_delta_rule(gi.q, gi.k, gi.v, gi.g, gi.beta, scale=gi.scale)[0]  # noqa: E731
        ops_ = {
            "gdn_op": op,
            "gdn_op_then_norm": lambda: rms_norm_gated(op(), og, ow, eps=1e-6),
            "gdn_op_norm_in_call": lambda: chunk_gated_delta_rule_gated_norm(gi.q, gi.k, gi.v, gi.g, gi.beta, og, ow,
                                                                              1e-6, scale=gi.scale)[0],
        }
        for name, fn in ops_.items():
            fn()
            settle(torch, fn)
            ms, _ = time_launches(torch, fn, steps)
            out[f"{name}_ms"] = round(ms, 4)
    pair_ms = out["gdn_layer_ms"] + out["attn_layer_ms"]
    out.update({
        "pair_ms": round(pair_ms, 4),
        "pair_tokens_per_s": round(B * T / (pair_ms * 1e-3), 1),
        "attn_kernel": "gated_attn_flash_fwd_kernel",
        "attn_kernel_ms": round(fa_ms, 4),
        "attn_flops": fl,
        "attn_tflops": round(fl / (fa_ms * 1e-3) / 1e12, 2),
        "attn_frac_mfma_peak": round(fl / (fa_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
    })
    return out


def time_launches(torch, fn, steps: int, indexed: bool = False) -> tuple[float, float]:
    """(mean ms per step from one event pair over all steps, mean ms per launch from per-launch event pairs).
    With `indexed`, call i is fn(i) (launches rotating over input sets)."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        starts[i].record(stream)
        fn(i) if indexed else fn()
        ends[i].record(stream)
    e1.record(stream)
    torch.cuda.synchronize()
    per_launch = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / steps
    return e0.elapsed_time(e1) / steps, per_launch


def time_back_to_back(torch, fn, steps: int, indexed: bool = False) -> float:
    """Mean ms per step from one event pair around `steps` back-to-back calls (no per-launch events).
    With `indexed`, call i is fn(i) (launches rotating over input sets)."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        fn(i) if indexed else fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


SETTLE_MS = 100.0  # default untimed run of a workload's own step before its warmup steps
_settle_ms = SETTLE_MS  # this process's value (--settle-ms)


def settle(torch, fn, ms: float | None = None) -> dict:
    """Runs `fn` untimed, back to back, for at least `ms` milliseconds (default: --settle-ms; a
    device sync every 8 calls).

    From idle this GPU's clocks take about 35 ms of this kind of load to settle: the first 50
    prefill steps of a fresh process run at ~157 us, the steady state at ~131 us. The same time
    spent on bf16 GEMMs or device copies does not settle them, and a 200 ms pause undoes it. The
    timed steps then measure the sustained rate a training or serving loop runs at; the prefill
    part also reports its first K steps without this phase."""
    ms = _settle_ms if ms is None else ms
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    calls = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            fn()
        calls += 8
        torch.cuda.synchronize()
    return {"calls": calls, "ms": round((time.perf_counter() - t0) * 1e3, 1)}


def launch_percentiles(torch, fn, steps: int) -> dict:
    """p10 / median / p90 of per-launch HIP-event times (ms), one event pair per launch."""
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        starts[i].record(stream)
        fn(i)
        ends[i].record(stream)
    torch.cuda.synchronize()
    ts = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    q = lambda f: ts[min(len(ts) - 1, int(round(f * (len(ts) - 1))))]
    return {"p10_ms": round(q(0.1), 4), "median_ms": round(q(0.5), 4), "p90_ms": round(q(0.9), 4)}


def capture_graph(torch, fn):
    """Capture fn (kernel launches on the current stream) into a CUDA/HIP graph after a side-stream warmup."""
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


def time_replays(torch, graph, n: int) -> float:
    """Mean ms per replay over n back-to-back replays (events on the replaying stream)."""
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(name)


def cpu_baseline(torch, decode_steps: int = 100, min_seconds: float = 12.0):
    """The CPU oracle timed on this host: config-1 prefill (full input), config-3's per-document loop
    (full input) and config-2 decode steps."""
    from oracle import decode_step_ref, recurrent_gated_delta_rule
    from sorernn_amd.synthetic import config_inputs, decode_inputs

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    inp = config_inputs(1)
    times = []
    start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - start < min_seconds and len(times) < 50):
        t0 = time.perf_counter()
        recurrent_gated_delta_rule(inp.q, inp.k, inp.v, inp.g, inp.beta, inp.scale, inp.h0, True)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    tokens = inp.q.shape[0] * inp.q.shape[1]
    # config 3: the oracle's per-document loop (one batch row, so every token step is a [1, 16, 128, 128]
    # update: ~10x slower per token than config 1's batch of 4); a bounded sample -- whole documents in
    # order until ~10 s have passed -- keeps the bench within minutes
    v3 = config_inputs(3)
    bounds = [int(x) for x in v3.cu_seqlens.tolist()]
    v_docs, v_tokens, v_t = 0, 0, 0.0
    for n, (a, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        cu1 = torch.tensor([0, e - a])
        t0 = time.perf_counter()
        recurrent_gated_delta_rule(v3.q[:, a:e], v3.k[:, a:e], v3.v[:, a:e], v3.g[:, a:e], v3.beta[:, a:e], v3.scale,
                                   v3.h0[n:n + 1], True, cu_seqlens=cu1)
        v_t += time.perf_counter() - t0
        v_docs, v_tokens = v_docs + 1, v_tokens + (e - a)
        if v_t >= 10.0:
            break
    di = decode_inputs()
    conv, st = di.conv_state.clone(), di.state.clone()
    t0 = time.perf_counter()
    for _ in range(decode_steps):
        _, conv, st = decode_step_ref(di.x_qkv, conv, di.conv_weight, di.g, di.beta, st, di.H, di.HV, di.D)
    dec_us = (time.perf_counter() - t0) / decode_steps * 1e6
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
    except Exception:
        pass
    return {
        "value": round(tokens / med, 1),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"full config-1 input (B=4, T=4096, H=16, d=128; 16384 tokens) through the oracle's torch fp32 "
                  f"recurrence, median of {len(times)} passes ({times[0]:.2f}-{times[-1]:.2f} s each, "
                  f"{sum(times):.1f} s total); decode: {decode_steps} config-2 steps incl. the conv cache; "
                  f"config 3: the per-document loop (varlen_config3)",
        "decode_us_per_step": round(dec_us, 1),
        "varlen_config3": {
            "tokens_per_s": round(v_tokens / v_t, 1),
            "sample": f"the first {v_docs} of config 3's 8 documents ({v_tokens} of {bounds[-1]} tokens, H=16, d=128, "
                      f"per-document h0 and final state) through the oracle's per-document loop, {v_t:.1f} s",
        },
        "cpu_model": cpu,
        "torch": torch.__version__,
        "host": platform.node(),
    }


def run_only(torch, args) -> int:
    """One workload for --steps launches (profiler runs: PMC counters per dispatch)."""
    from sorernn_amd import chunk_gated_delta_rule, gated_delta_decode_step
    from sorernn_amd.synthetic import config_inputs, decode_inputs

    if args.only == "block_pair":
        bp = block_pair(torch, args.steps)
        print(f"ran block_pair: gdn {bp['gdn_layer_ms']} ms (chunk op and norm as two calls {bp['gdn_layer_unfused_epilogue_ms']} ms, "
              f"reference route {bp['gdn_layer_reference_route_ms']} ms), attn {bp['attn_layer_ms']} ms, "
              f"attention kernel {bp['attn_kernel_ms']} ms; GDN call {bp['gdn_op_ms']} ms, then the norm kernel "
              f"{bp['gdn_op_then_norm_ms']} ms, norm in the call {bp['gdn_op_norm_in_call_ms']} ms", flush=True)
        return 0
    if args.only in ("gdn_norm_call", "gdn_norm_two_calls"):
        # config 4's GDN call with the layer's gated RMSNorm: in the call (the layer's route), or the
        # op followed by the norm kernel; synthetic config-1 distributions, bf16 gate, --steps calls
        from sorernn_amd import rms_norm_gated
        from sorernn_amd.ops import chunk_gated_delta_rule_gated_norm
        from sorernn_amd.synthetic import gdn_inputs
        gi = gdn_inputs(2, 8192, 16, 128, dtype=torch.bfloat16, seed=1004).to("cuda")
        og = torch.randn(2, 8192, 16, 128, device="cuda").to(torch.bfloat16)
        ow = torch.rand(128, device="cuda") + 0.5
        for _ in range(args.steps):
            if args.only == "gdn_norm_call":
                chunk_gated_delta_rule_gated_norm(gi.q, gi.k, gi.v, gi.g, gi.beta, og, ow, 1e-6, scale=gi.scale)
            else:
                o, _ = chunk_gated_delta_rule(gi.q, gi.k, gi.v, gi.g, gi.beta, scale=gi.scale)
                rms_norm_gated(o, og, ow, eps=1e-6)
        torch.cuda.synchronize()
        print(f"ran {args.only}: {args.steps} calls", flush=True)
        return 0
    if args.only == "train":
        tf, tb = train_step_times(torch, config_inputs(1).to("cuda"), args.steps)
        print(f"ran train: {args.steps} steps, forward {tf:.3f} ms, backward {tb:.3f} ms", flush=True)
        return 0
    if args.only == "varlen_docs":
        _, cu_cpu, inp = varlen_docs_inputs(torch)
        d = inp.to("cuda")

        def step(i):
            chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, cu_seqlens=d.cu_seqlens,
                                   cu_seqlens_cpu=cu_cpu)
    elif args.only in ("prefill", "varlen"):
        # as in the bench: launches alternate over two input sets
        idx = 1 if args.only == "prefill" else 3
        inp = config_inputs(idx)
        cu_cpu = inp.cu_seqlens
        d = inp.to("cuda")
        sets = rotating_sets(d)

        def step(i):
            q_, k_, v_, g_, b_, h_ = sets[i % len(sets)]
            chunk_gated_delta_rule(q_, k_, v_, g_, b_, scale=d.scale, initial_state=h_,
                                   output_final_state=True, cu_seqlens=d.cu_seqlens, cu_seqlens_cpu=cu_cpu)
    else:
        di = decode_inputs()
        x, cs, cw, g, b, st = (t.to("cuda") for t in (di.x_qkv, di.conv_state, di.conv_weight, di.g, di.beta, di.state))
        # decode_rot: 5 state/conv copies visited in turn (335 MB > the 256 MB Infinity Cache), so the
        # profiled steps read their state from DRAM
        nrot = 5 if args.only == "decode_rot" else 1
        states = [st] + [st.clone() for _ in range(nrot - 1)]
        convs = [cs] + [cs.clone() for _ in range(nrot - 1)]

        def step(i):
            gated_delta_decode_step(x, convs[i % nrot], cw, g, b, states[i % nrot], di.H, di.HV, di.D)
    # as in the bench: the workload's own step untimed for the settle time, then W + K launches (the
    # last K of a trace are the ones the bench times)
    st_ = settle(torch, lambda: [step(i) for i in range(2)])
    for i in range(args.warmup + args.steps):
        step(i)
    torch.cuda.synchronize()
    print(f"ran {args.only}: {st_['calls']} settle launches, then {args.warmup + args.steps} launches", flush=True)
    return 0


PARTS = ("prefill", "decode", "varlen", "varlen_docs", "train", "block_pair")
DOC_LENGTHS = os.path.join(ROOT, "tests", "golden", "doc_lengths_pt.json")


def doc_length_windows() -> list[list[int]]:
    """Document lengths of the real-distribution leg: 8 windows of 4,096 tokens filled with lengths
    drawn from the reference's Portuguese-corpus sample (data/sample_pt/doc_lengths.json, sampled by
    tests/golden/make_doc_lengths.py as the reference's bench --doc-lengths does)."""
    with open(DOC_LENGTHS) as f:
        return json.load(f)["windows"]


def varlen_docs_inputs(torch):
    """Lengths, host cu_seqlens and seeded inputs of the real-distribution leg (one packed batch row)."""
    from sorernn_amd.synthetic import gdn_inputs

    lens = [n for w in doc_length_windows() for n in w]
    cu = torch.tensor([0] + list(itertools.accumulate(lens)), dtype=torch.long)
    return lens, cu, gdn_inputs(1, int(cu[-1]), 16, 128, dtype=torch.bfloat16, seed=1005, h0=False, cu_seqlens=cu)


def rotating_sets(inp, n: int = 2):
    """`n` copies of a workload's device inputs (the first is `inp`'s own tensors), visited in turn so
    that no launch finds its inputs left in the 256 MB Infinity Cache by the previous one: every
    config-1 set (q, k, v, g, beta, h0 and the outputs it writes) is 281 MB."""
    base = (inp.q, inp.k, inp.v, inp.g, inp.beta, inp.h0)
    return [base] + [tuple(None if x is None else x.clone() for x in base) for _ in range(n - 1)]


def part_prefill(torch, args) -> dict:
    """Config 1: the chunked prefill op, events around every launch.

    The headline (`ms_step`, `ms_launch`, the percentiles) comes from launches alternating over two
    input sets (2 x 281 MB, more than the 256 MB Infinity Cache), so every launch reads its inputs
    from DRAM, as the layers of a model do; the same figures with one input set, whose inputs the
    previous launch leaves in the Infinity Cache, are reported beside them (`*_cache_resident`)."""
    from sorernn_amd import chunk_gated_delta_rule
    from sorernn_amd.synthetic import config_inputs

    inp = config_inputs(1).to("cuda")
    B, T, H, K = inp.q.shape
    sets = rotating_sets(inp)

    def step_rot(i):
        q_, k_, v_, g_, b_, h_ = sets[i % len(sets)]
        return chunk_gated_delta_rule(q_, k_, v_, g_, b_, scale=inp.scale, initial_state=h_, output_final_state=True)

    def step():
        return step_rot(0)

    for i in range(args.warmup):
        step_rot(i)
    torch.cuda.synchronize()
    # the first K steps of the process after W warmup steps (reported beside the headline)
    cold_ms = time_back_to_back(torch, step_rot, args.steps, indexed=True)
    st = settle(torch, lambda: [step_rot(i) for i in range(len(sets))])
    for i in range(args.warmup):
        step_rot(i)
    torch.cuda.synchronize()
    # the step rate from back-to-back calls with events only around the whole run; the per-launch
    # (op) times from a second run with an event pair around every call
    t0 = time.perf_counter()
    ms_step = time_back_to_back(torch, step_rot, args.steps, indexed=True)
    wall = (time.perf_counter() - t0) / args.steps * 1e3
    _, ms_launch = time_launches(torch, step_rot, args.steps, indexed=True)
    pct = launch_percentiles(torch, step_rot, args.steps)
    # one input set, launch after launch: its inputs stay in the Infinity Cache
    ms_step_c = time_back_to_back(torch, step, args.steps)
    _, ms_launch_c = time_launches(torch, step, args.steps)
    pct_c = launch_percentiles(torch, lambda i: step(), args.steps)
    return {"B": B, "T": T, "H": H, "K": K, "ms_step": ms_step, "ms_launch": ms_launch, "wall_ms": wall,
            "pct": pct, "ms_step_cache_resident": ms_step_c, "ms_launch_cache_resident": ms_launch_c,
            "pct_cache_resident": pct_c, "input_sets": len(sets), "cold_ms_step": cold_ms, "settle": st,
            "min_bytes": 4 * inp.q.numel() * 2 + 2 * inp.g.numel() * 4 + 2 * inp.h0.numel() * 4}


def part_decode(torch, args) -> dict:
    """Config 2: the fused decode step. The step is captured once into a HIP graph and replayed back
    to back (a serving loop launches the same fixed-shape step every token); the eager,
    host-launched rate is reported beside it, and a run rotating over 5 state copies forces DRAM."""
    from sorernn_amd import gated_delta_decode_step
    from sorernn_amd.synthetic import decode_inputs

    dev = "cuda"
    di = decode_inputs()
    x, cs, cw, g, b, st = (t.to(dev) for t in (di.x_qkv, di.conv_state, di.conv_weight, di.g, di.beta, di.state))
    out = torch.empty(di.x_qkv.shape[0], 1, di.HV, di.D, device=dev, dtype=di.x_qkv.dtype)

    def dstep(state=st, conv=cs):
        gated_delta_decode_step(x, conv, cw, g, b, state, di.H, di.HV, di.D, out=out)

    for _ in range(10):
        dstep()
    settle(torch, dstep)
    # eager: host-launched steps back to back, one event pair around the run (events around every
    # step would add their own host time, which a serving loop does not pay); the host time per call
    # is measured beside it with the device left to drain
    n_eager = min(args.decode_steps, 200)
    eager_ms = time_back_to_back(torch, dstep, n_eager)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_eager):
        dstep()
    host_us = (time.perf_counter() - t0) / n_eager * 1e6
    torch.cuda.synchronize()
    per_graph = 50  # steps per captured graph: one graph launch per 50 steps keeps the host off the critical path

    def dsteps():
        for _ in range(per_graph):
            dstep()

    graph = capture_graph(torch, dsteps)
    dec_ms = time_replays(torch, graph, max(1, args.decode_steps // per_graph)) / per_graph
    nrot = 5
    states = [st.clone() for _ in range(nrot)]
    convs = [cs.clone() for _ in range(nrot)]

    def dstep_rot():
        for _ in range(per_graph // nrot):
            for i in range(nrot):
                dstep(states[i], convs[i])

    rgraph = capture_graph(torch, dstep_rot)
    rot_ms = time_replays(torch, rgraph, max(1, args.decode_steps // per_graph)) / per_graph
    torch.cuda.synchronize()
    return {"us_step": dec_ms * 1e3, "rot_us_step": rot_ms * 1e3, "eager_us_step": eager_ms * 1e3,
            "eager_host_us_per_call": host_us, "per_graph": per_graph}


def part_varlen(torch, args) -> dict:
    """Config 3: 8 packed documents, 32768 tokens, per-document initial and final states; launches
    alternate over two input sets (one set is 536 MB of q, k, v and o: more than the Infinity Cache
    already, the second set makes that hold whatever the outputs' placement)."""
    from sorernn_amd import chunk_gated_delta_rule
    from sorernn_amd.synthetic import config_inputs

    v3 = config_inputs(3)
    cu_cpu = v3.cu_seqlens
    v3 = v3.to("cuda")
    sets = rotating_sets(v3)

    def vstep(i):
        q_, k_, v_, g_, b_, h_ = sets[i % len(sets)]
        return chunk_gated_delta_rule(q_, k_, v_, g_, b_, scale=v3.scale, initial_state=h_,
                                      output_final_state=True, cu_seqlens=v3.cu_seqlens, cu_seqlens_cpu=cu_cpu)

    for i in range(3):
        vstep(i)
    settle(torch, lambda: [vstep(i) for i in range(len(sets))])
    n = max(6, args.steps // 5)
    v_ms, v_launch = time_launches(torch, vstep, n, indexed=True)
    v_pct = launch_percentiles(torch, vstep, n)
    return {"ms_step": v_ms, "ms_launch": v_launch, "pct": v_pct, "lens": (cu_cpu[1:] - cu_cpu[:-1]).tolist(),
            "input_sets": len(sets)}


def part_varlen_docs(torch, args) -> dict:
    """The reference model's call on its real document-length distribution: 8 windows of 4,096 tokens
    packed into one batch row (53 documents, lengths from the committed fixture), H=16, d=128, bf16
    q/k/v, fp32 g/beta as in config 1, zero initial state and no final state (sore/model/gdn.py:166-169
    discards it)."""
    from sorernn_amd import chunk_gated_delta_rule

    lens, cu, inp = varlen_docs_inputs(torch)
    d = inp.to("cuda")

    def step():
        return chunk_gated_delta_rule(d.q, d.k, d.v, d.g, d.beta, scale=inp.scale, cu_seqlens=d.cu_seqlens,
                                      cu_seqlens_cpu=cu)

    for _ in range(3):
        step()
    settle(torch, step)
    n = max(5, args.steps // 5)
    ms, launch = time_launches(torch, step, n)
    pct = launch_percentiles(torch, lambda i: step(), n)
    return {"ms_step": ms, "ms_launch": launch, "pct": pct, "lens": lens}


def part_train(torch, args) -> dict:
    """Config 1 under autograd: the training forward and the backward, timed separately."""
    from sorernn_amd.synthetic import config_inputs

    inp = config_inputs(1).to("cuda")
    tf, tb = train_step_times(torch, inp, max(5, args.steps // 5))
    return {"fwd_ms": tf, "bwd_ms": tb}


def part_block_pair(torch, args) -> dict:
    return block_pair(torch, max(5, args.steps // 5))


PART_FNS = {"prefill": part_prefill, "decode": part_decode, "varlen": part_varlen, "varlen_docs": part_varlen_docs,
            "train": part_train, "block_pair": part_block_pair}


def varlen_docs_entry(vd: dict) -> dict:
    lens = vd["lens"]
    fl = chunk_flops(lens, 16, 128)
    srt = sorted(lens)
    return {
        "workload": f"reference document-length distribution: 8 windows of 4096 tokens, {len(lens)} packed docs "
                    f"(median {srt[len(srt) // 2]}, max {srt[-1]}; tests/golden/doc_lengths_pt.json), H=16, d=128, "
                    "zero h0, no final state",
        "tokens_per_s": round(sum(lens) / (vd["ms_step"] * 1e-3), 1),
        "ms_per_launch": round(vd["ms_launch"], 4),
        "launch_percentiles": vd["pct"],
        "tflops": round(fl / (vd["ms_launch"] * 1e-3) / 1e12, 2),
        "frac_mfma_peak": round(fl / (vd["ms_launch"] * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "longest_doc_chunks": -(-srt[-1] // C),
    }


def assemble(parts: dict, args, cpu: dict | None) -> dict:
    """The one JSON line from the workloads' raw measurements (no GPU work here)."""
    pf, dc, vl, tr = parts["prefill"], parts["decode"], parts["varlen"], parts["train"]
    B, T, H, K = pf["B"], pf["T"], pf["H"], pf["K"]
    ms_step, ms_launch = pf["ms_step"], pf["ms_launch"]
    flops = chunk_flops([T] * B, H, K)
    flops_c = chunk_flops_causal([T] * B, H, K)
    achieved = flops / (ms_launch * 1e-3) / 1e12
    tparts = [load_traffic(k) for k in PREFILL_KERNELS]
    traffic = sum(tparts) if all(x is not None for x in tparts) else None
    dbytes = decode_bytes()
    dec_s, rot_s = dc["us_step"] * 1e-6, dc["rot_us_step"] * 1e-6
    lens = vl["lens"]
    v_flops = chunk_flops(lens, 16, 128)
    b_flops = chunk_bwd_flops([T] * B, H, K)
    tr_f, tr_b = tr["fwd_ms"], tr["bwd_ms"]
    result = {
        "metric": "GDN prefill tokens/s & decode-step µs (H=16,d=128); % of MI355X roofline",
        "value": round(B * T / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "wall_ms_per_step": round(pf["wall_ms"], 4),
        "cold_ms_per_step": round(pf["cold_ms_step"], 4) if "cold_ms_step" in pf else None,
        "cold_value": round(B * T / (pf["cold_ms_step"] * 1e-3), 1) if "cold_ms_step" in pf else None,
        "cache_resident_ms_per_step": round(pf["ms_step_cache_resident"], 4),
        "cache_resident_value": round(B * T / (pf["ms_step_cache_resident"] * 1e-3), 1),
        "timing": "value / ms_per_step: back-to-back launches alternating over two input sets (2 x 281 MB > the "
                  "256 MB Infinity Cache), one event pair around the run; cache_resident_*: the same with one "
                  "input set",
        "settle": {"ms_per_workload": args.settle_ms, "prefill_calls": pf.get("settle", {}).get("calls"),
                   "note": "every workload runs its own step untimed, back to back, for >= settle ms before "
                           "its W warmup steps (from idle the GPU's clocks settle after ~35 ms of this load); "
                           "cold_ms_per_step / cold_value are the process's first K prefill steps after W "
                           "warmup steps, without the settle phase"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded CPU generator, BASELINE config 1 distributions)",
        "config": {"workload": "config1 chunked GDN prefill: B=4, T=4096, H=HV=16, d_k=d_v=128, chunk=64, "
                               "bf16 q/k/v, fp32 g/beta/h0, output_final_state",
                   "global_batch": B, "seq_len": T, "parallelism": "single GPU"},
        "roofline": {
            "bound": "mfma",
            "kernel": " + ".join(PREFILL_KERNELS),
            "achieved": round(achieved, 2),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "flops_per_launch": flops,
            "min_hbm_bytes_per_launch": pf["min_bytes"],
            "hbm_frac_at_min_bytes": round(pf["min_bytes"] / (ms_launch * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "ms_per_launch": round(ms_launch, 4),
            "launch_percentiles": pf["pct"],
            "input_sets": pf["input_sets"],
            "timing": "launches alternating over two input sets (2 x 281 MB > the 256 MB Infinity Cache): every "
                      "launch reads its inputs from DRAM",
            "cache_resident_ms_per_launch": round(pf["ms_launch_cache_resident"], 4),
            "cache_resident_achieved": round(flops / (pf["ms_launch_cache_resident"] * 1e-3) / 1e12, 2),
            "cache_resident_frac": round(flops / (pf["ms_launch_cache_resident"] * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "cache_resident_launch_percentiles": pf["pct_cache_resident"],
            "cache_resident_note": "one input set, launch after launch: the previous launch leaves the inputs in "
                                   "the Infinity Cache",
            # secondary FLOP conventions: causal tiles only (5C^2d + 6Cd^2 per chunk-head), and the
            # reference's flops.py count of 4*K*V per token-head
            "flops_causal_halved": flops_c,
            "frac_causal_halved": round(flops_c / (ms_launch * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "flops_reference_flops_py": 4 * K * K * B * T * H,
        },
        "decode": {
            "workload": "config2: B=64, H=HV=16, D=128, conv cache [64,6144,4] bf16, fp32 state updated in place; "
                        "headline figures with the state served from DRAM",
            "kernel": "gated_delta_decode_w4_kernel",
            "us_per_step": round(dc["rot_us_step"], 3),
            "timing": f"{args.decode_steps} back-to-back fused steps: replays of a HIP graph holding "
                      f"{dc['per_graph']} steps, visiting 5 state/conv copies in turn (5 x 73 MB > the 256 MB "
                      "Infinity Cache), so every step reads its state from DRAM",
            "bytes_per_step": dbytes,
            "achieved_GBs": round(dbytes / rot_s / 1e9, 1),
            "frac_hbm_peak": round(dbytes / rot_s / 1e9 / HBM_PEAK_GBS, 4),
            "cache_resident_us_per_step": round(dc["us_step"], 3),
            "cache_resident_note": "one state and conv cache, updated in place step after step: the 73 MB stay in "
                                   "the Infinity Cache",
            "cache_resident_frac_hbm_peak": round(dbytes / dec_s / 1e9 / HBM_PEAK_GBS, 4),
            "eager_us_per_step": round(dc["eager_us_step"], 3),
            "eager_host_us_per_call": round(dc.get("eager_host_us_per_call", float("nan")), 2),
            "eager_note": "host-launched steps back to back on one state (compare cache_resident_us_per_step); "
                          "eager_host_us_per_call is the Python + launch time of one call",
            "steps": args.decode_steps,
        },
        "varlen": {
            "workload": "config3: 8 packed docs, 32768 tokens, H=16, d=128, per-doc h0 and final states",
            "doc_lengths": lens,
            "tokens_per_s": round(32768 / (vl["ms_step"] * 1e-3), 1),
            "ms_per_launch": round(vl["ms_launch"], 4),
            "launch_percentiles": vl["pct"],
            "tflops": round(v_flops / (vl["ms_launch"] * 1e-3) / 1e12, 2),
            "frac_mfma_peak": round(v_flops / (vl["ms_launch"] * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "input_sets": vl.get("input_sets", 1),
        },
        "varlen_docs": varlen_docs_entry(parts["varlen_docs"]),
        "train": {
            "workload": "config1 under autograd: training forward (saves bf16 per-chunk states) + backward "
                        "(dq, dk, dv, dg, dbeta, dh0) of chunk_gated_delta_rule",
            "fwd_ms": round(tr_f, 4),
            "bwd_ms": round(tr_b, 4),
            "tokens_per_s_fwd_bwd": round(B * T / ((tr_f + tr_b) * 1e-3), 1),
            "bwd_flops": b_flops,
            "bwd_tflops": round(b_flops / (tr_b * 1e-3) / 1e12, 2),
            "bwd_frac_mfma_peak": round(b_flops / (tr_b * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "kernels": "gated_delta_chunk_kernel<SAVE>; gated_delta_chunk_bwd_prep_kernel, "
                       "gated_delta_chunk_bwd_state_kernel, gated_delta_chunk_bwd_grad_kernel",
        },
        "block_pair": parts["block_pair"],
        "isolation": "each workload ran in its own child process (a fresh HIP context and allocator)",
    }
    if cpu is not None:
        result["cpu_baseline"] = cpu
    return result


def run_part(part: str, args) -> dict:
    """Run one workload in a child process and return the JSON object it prints last. Its stderr
    (progress) passes through; a failing child ends the bench with the child's status."""
    cmd = [sys.executable, "-u", os.path.abspath(__file__), "--part", part, "--steps", str(args.steps),
           "--warmup", str(args.warmup), "--decode-steps", str(args.decode_steps), "--settle-ms", str(args.settle_ms)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, text=True)
    if res.returncode != 0:
        print(f"bench.py: workload {part} failed (status {res.returncode}); output:\n{res.stdout}", file=sys.stderr)
        raise SystemExit(res.returncode if res.returncode > 0 else 1)
    lines = [ln for ln in res.stdout.splitlines() if ln.strip()]
    if not lines:
        print(f"bench.py: workload {part} printed nothing", file=sys.stderr)
        raise SystemExit(1)
    return json.loads(lines[-1])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (the reference kernel for PMC byte counters)")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed run of each workload's own step before its warmup steps (0: none)")
    ap.add_argument("--only", choices=list(PARTS) + ["decode_rot", "gdn_norm_call", "gdn_norm_two_calls"], default=None,
                    help="run one workload only (for profiler runs); prints no JSON line")
    ap.add_argument("--part", choices=PARTS, default=None,
                    help="(internal) run one workload and print its raw measurements as JSON")
    args = ap.parse_args()
    global _settle_ms
    _settle_ms = args.settle_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build runs one GPU only (the GDN op needs no collective: every (sequence, head) "
              f"chain is independent); got --gpus {args.gpus}. Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if args.part or args.only or args.calibrate_copy:
        if not torch.cuda.is_available():
            print("bench.py: no GPU visible", file=sys.stderr)
            return 1
        if args.calibrate_copy:
            # 256 MiB read + 256 MiB written per launch: divides FETCH_SIZE / WRITE_SIZE into a scale factor
            src = torch.empty(64 * 1024 * 1024, device="cuda", dtype=torch.float32).fill_(1.0)
            dst = torch.empty_like(src)
            for _ in range(args.steps):
                dst.copy_(src)
            torch.cuda.synchronize()
            print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "launches": args.steps}))
            return 0
        if args.only:
            return run_only(torch, args)
        out = PART_FNS[args.part](torch, args)
        torch.cuda.synchronize()
        print(f"bench.py: {args.part} done", file=sys.stderr, flush=True)
        print(json.dumps(out), flush=True)
        return 0
    # The full run: every workload in its own child process (this process never touches the GPU;
    # counting devices does not initialise it), then the CPU baseline here.
    if torch.cuda.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    parts = {}
    for part in PARTS:
        parts[part] = run_part(part, args)
    cpu = None if args.no_cpu_baseline else cpu_baseline(torch)
    print(json.dumps(assemble(parts, args, cpu)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
