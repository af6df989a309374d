"""CPU checks of the C ABI: libgdn.so loads, exports every entry point of include/gdn.h with the
parameter counts the ctypes binding declares, and the host layer rejects bad calls before any launch.
"""
import os
import re

import pytest
import torch

from sorernn_amd import _lib
from sorernn_amd import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gdn.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"GDN_API\s+[\w\s\*]+?\b(gdn_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_header_declares_the_entry_points():
    decl = _declared()
    assert set(decl) == set(_lib.SIGNATURES), f"header {sorted(decl)} vs binding {sorted(_lib.SIGNATURES)}"


def test_library_exports_every_declared_symbol_with_matching_arity():
    lib = _lib.load()
    for name, nparams in _declared().items():
        assert hasattr(lib, name), f"{name} not exported by libgdn.so"
        assert len(_lib.SIGNATURES[name]) == nparams, f"{name}: binding has {len(_lib.SIGNATURES[name])} params, header {nparams}"
    assert lib.gdn_abi_version() == _lib.ABI_VERSION


def test_set_range_flag_checks_the_device_first():
    """gdn_set_range_flag validates the device index before any HIP call (no GPU needed)."""
    lib = _lib.load()
    assert lib.gdn_set_range_flag(-1, None) == _lib.GDN_ERR_INVALID
    assert b"out of range" in lib.gdn_last_error()
    assert lib.gdn_set_range_flag(64, None) == _lib.GDN_ERR_INVALID


def test_no_cpu_path():
    q = torch.randn(1, 4, 1, 64)
    with pytest.raises(ValueError, match="GPU"):
        chunk_gated_delta_rule(q, q, q, torch.zeros(1, 4, 1), torch.ones(1, 4, 1))
    with pytest.raises(ValueError, match="GPU"):
        fused_recurrent_gated_delta_rule(q, q, q, torch.zeros(1, 4, 1), torch.ones(1, 4, 1))


def test_unsupported_options_raise():
    q = torch.randn(1, 4, 1, 64)
    with pytest.raises(NotImplementedError):
        chunk_gated_delta_rule(q, q, q, torch.zeros(1, 4, 1), torch.ones(1, 4, 1), allow_neg_eigval=True)


def _align(b):
    return (b + 255) // 256 * 256


def _coop_front(t, hv, n):
    """The cooperative prefill's package ring (47,360 bytes per slot: the fp16 K and Q rows, P, the T/A
    blocks and the gate terms of a chunk; min(8, ceil(T / 64)) slots per (sequence, head) chain) and its
    sync words (8 + 8 per slot of 8 per chain, 4 bytes each, plus one error word)."""
    slots = min(8, max(1, -(-t // 64)))
    return _align(n * hv * slots * 47360) + _align((n * hv * (8 + 8 * 8) + 1) * 4)


def test_chunk_workspace_size_matches_layout(monkeypatch):
    """gdn_chunk_workspace_size: the two-kernel prefill's T - I rows (one 128-byte row per token-head),
    or, while SORERNN_PREFILL=coop selects the cooperative prefill, the larger of those and its package
    ring + sync words; plus the varlen index arrays (chunk_first[N + 1] and order[N], int32, 256-byte
    aligned each); 0 for invalid sizes."""
    from sorernn_amd.ops import chunk_workspace_bytes
    monkeypatch.delenv("SORERNN_PREFILL", raising=False)
    assert chunk_workspace_bytes(4, 4096, 16, 4, False) == 4 * 4096 * 16 * 128
    assert chunk_workspace_bytes(1, 32768, 16, 8, True) == 32768 * 16 * 128 + 512
    # Many short documents: the ring would need 300 x 3 x 2 slots of 47,360 bytes, the rows only 38 KB.
    assert chunk_workspace_bytes(1, 100, 3, 300, True) == _align(100 * 3 * 128) + 2560
    assert chunk_workspace_bytes(0, 100, 3, 1, False) == 0
    monkeypatch.setenv("SORERNN_PREFILL", "coop")
    assert chunk_workspace_bytes(4, 4096, 16, 4, False) == max(4 * 4096 * 16 * 128, _coop_front(4096, 16, 4))
    assert chunk_workspace_bytes(4, 4096, 16, 4, False) == 4 * 4096 * 16 * 128
    assert chunk_workspace_bytes(1, 32768, 16, 8, True) == max(32768 * 16 * 128, _coop_front(32768, 16, 8)) + 512
    assert chunk_workspace_bytes(1, 100, 3, 300, True) == _coop_front(100, 3, 300) + 2560
    assert chunk_workspace_bytes(0, 100, 3, 1, False) == 0


def test_gated_norm_workspace_size_matches_layout(monkeypatch):
    """gdn_chunk_gated_norm_workspace_size: gdn_chunk_fwd's workspace, then the epilogue's progress
    words (a 256-byte block per (sequence, value head)); 0 for invalid sizes or head dims."""
    from sorernn_amd import _lib
    from sorernn_amd.ops import chunk_workspace_bytes
    monkeypatch.delenv("SORERNN_PREFILL", raising=False)
    lib = _lib.load()
    for (b, t, hv, n, v, varlen) in [(2, 8192, 16, 2, 128, 0), (1, 777, 4, 5, 128, 1), (2, 300, 2, 2, 64, 0)]:
        assert lib.gdn_chunk_gated_norm_workspace_size(b, t, hv, n, v, varlen) == (
            chunk_workspace_bytes(b, t, hv, n, bool(varlen)) + _align(n * hv * 256))
    assert lib.gdn_chunk_gated_norm_workspace_size(2, 300, 2, 2, 96, 0) == 0
    assert lib.gdn_chunk_gated_norm_workspace_size(0, 300, 2, 2, 128, 0) == 0


def test_chunk_backward_buffer_sizes_match_layout():
    """gdn_chunk_states_size: one bf16 K x V state per chunk and value head (chunk count bounded by
    ceil(T/64) + N with cu_seqlens). gdn_chunk_bwd_workspace_size: bf16 (T - I)^T rows [tokens][HV][64],
    bf16 G1 [chunks][HV][V][64], bf16 dS' per chunk [chunks][HV][V][K] and two fp32 partial sums per
    chunk-head, each 256-byte aligned."""
    lib = _lib.load()
    a = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert lib.gdn_chunk_states_size(4, 4096, 16, 128, 128, 4, 0) == 4 * 64 * 16 * 128 * 128 * 2
    assert lib.gdn_chunk_states_size(1, 100, 3, 64, 64, 5, 1) == (2 + 5) * 3 * 64 * 64 * 2
    tok, ch = 4 * 4096, 4 * 64
    assert lib.gdn_chunk_bwd_workspace_size(4, 4096, 16, 128, 128, 4, 0) == (
        a(tok * 16 * 128) + a(ch * 16 * 128 * 64 * 2) + a(ch * 16 * 128 * 128 * 2) + a(ch * 16 * 8))
    tok, ch = 100, 2 + 5  # varlen: the chunk bound ceil(T/64) + N sizes G1
    assert lib.gdn_chunk_bwd_workspace_size(1, 100, 3, 64, 64, 5, 1) == (
        a(tok * 3 * 128) + a(ch * 3 * 64 * 64 * 2) + a(ch * 3 * 64 * 64 * 2) + a(ch * 3 * 8))
    assert lib.gdn_chunk_bwd_workspace_size(0, 4096, 16, 128, 128, 4, 0) == 0


def _kernel_names(files):
    csrc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "sorernn_amd", "csrc")
    names = []
    for f in sorted(os.listdir(csrc)):
        if f.endswith(".hip") and files(f):
            src = open(os.path.join(csrc, f)).read()
            names += re.findall(r"__global__\s+(?:__launch_bounds__\([^)]*\)\s+)?void\s+(\w+)", src)
    return names


# The reference profiler's rules in precedence order (sore/train/profiling.py:33-40): a kernel name
# lands in the first category whose regex it matches.
_PROFILER_RULES = (
    ("gdn", r"^(chunk_|recompute_w_u|prepare_wy_repr|l2norm_|fused_recurrent|fused_gdn|solve_tril|merge_16x16|causal_conv1d)|gated_delta"),
    ("attention", r"flex_attention|fmha_|flash_(fwd|bwd)|pytorch_flash|efficient_attention"),
    ("loss", r"nll_loss|log_softmax|LogSoftMax|SoftMax(Forward|Backward)|softmax_warp|cross_entropy"),
    ("matmul", r"gemm|gemv|cutlass|cublas|xmma|nvjet|^triton_tem_"),
    ("elementwise", r"^triton_(poi|red|per)_|elementwise_kernel|reduce_kernel|multi_tensor_apply|CatArrayBatchedCopy|index_elementwise|gather_kernel|indexSelect|lpnorm|embedding_backward"),
)


def _category(name: str) -> str:
    for cat, pat in _PROFILER_RULES:
        if re.search(pat, name):
            return cat
    return "other"


def test_every_kernel_name_matches_the_reference_profiler_gdn_rule():
    """The reference's profiler files kernels by name (sore/train/profiling.py:33-40). Every kernel of
    the GDN path lands in "gdn"; the attention layer's flash kernel in "attention" and its q/k
    norm + rotary prologue in "elementwise" (where the reference's torch ops for it land)."""
    gdn = _kernel_names(lambda f: not f.startswith("attn"))
    assert len(gdn) >= 15, gdn
    for n in gdn:
        assert _category(f"void gdn::{n}<128, 128>(gdn::Params)") == "gdn", n
    attn = _kernel_names(lambda f: f.startswith("attn"))
    cats = {n: _category(f"void gdn::{n}<128>(gdn::AttnParams)") for n in attn}
    assert cats == {"gated_attn_qk_norm_rope_elementwise_kernel": "elementwise",
                    "gated_attn_flash_fwd_kernel": "attention"}, cats


def test_gated_attention_layer_keeps_the_reference_parameter_names():
    """GatedAttention's state_dict keys and shapes (sore/model/attention.py:83-91)."""
    from sorernn_amd.attention import AttnLayerConfig, GatedAttention

    layer = GatedAttention(AttnLayerConfig(d_model=256, attn_heads=4, attn_kv_heads=2, attn_head_dim=64))
    shapes = {n: tuple(p.shape) for n, p in layer.state_dict().items()}
    assert shapes == {"q_proj.weight": (256, 256), "gate_proj.weight": (256, 256), "k_proj.weight": (128, 256),
                      "v_proj.weight": (128, 256), "q_norm.weight": (64,), "k_norm.weight": (64,),
                      "o_proj.weight": (256, 256)}
    assert layer.rotary.rot_dim == 16
    with pytest.raises(ValueError, match="rot_dim"):
        GatedAttention(AttnLayerConfig(d_model=64, attn_head_dim=6, rope_partial=0.5))
    with pytest.raises(ValueError, match="B == 1"):
        with torch.no_grad():
            layer(torch.zeros(2, 3, 256), torch.tensor([0, 3]))
