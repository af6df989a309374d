"""ctypes binding of ``libgdn.so`` (the C ABI declared in ``include/gdn.h``).

The library is loaded after ``torch`` so that it shares torch's HIP runtime (both resolve the
soname ``libamdhip64.so.7``): the stream handles torch hands out are then valid in the library.
A missing library is an error; nothing in this package computes the path on the CPU.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (load torch's HIP runtime first)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgdn.so")

GDN_OK = 0
GDN_ERR_INVALID, GDN_ERR_UNSUPPORTED, GDN_ERR_HIP = 1, 2, 3
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
FLAG_QK_L2NORM = 0x1
FLAG_BETA_SIGMOID = 0x2
FLAG_GATE_IN_KERNEL = 0x4
FLAG_CU_INT32 = 0x8
ACT_NONE, ACT_SILU, ACT_SILU_ROUNDED = 0, 1, 2
ABI_VERSION = 7

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F = ctypes.c_float
_U = ctypes.c_uint
_SZ = ctypes.c_size_t

# name -> argtypes, mirroring include/gdn.h
SIGNATURES = {
    "gdn_abi_version": [],
    "gdn_last_error": [],
    "gdn_chunk_fwd": [_P] * 9 + [_I64] * 7 + [_INT] * 3 + [_F, _U, _P, _P, _P, _SZ, _P],
    "gdn_chunk_workspace_size": [_I64] * 4 + [_INT],
    "gdn_chunk_fwd_gated_norm": [_P] * 9 + [_I64] * 7 + [_INT] * 3 + [_F, _U, _P, _P, _P, _P, _F, _INT, _P, _SZ, _P],
    "gdn_chunk_gated_norm_workspace_size": [_I64] * 5 + [_INT],
    "gdn_chunk_fwd_train": [_P] * 9 + [_I64] * 7 + [_INT] * 3 + [_F, _U, _P, _P, _P, _P, _SZ, _P],
    "gdn_chunk_fwd_noalloc": [_P] * 9 + [_I64] * 7 + [_INT] * 3 + [_F, _U, _P, _P, _P],
    "gdn_chunk_fwd_noalloc_max_workspace": [],
    "gdn_set_range_flag": [_INT, _P],
    "gdn_chunk_states_size": [_I64] * 6 + [_INT],
    "gdn_chunk_bwd": [_P] * 10 + [_I64] * 7 + [_INT] * 3 + [_F, _U] + [_P] * 11 + [_SZ, _P],
    "gdn_chunk_bwd_workspace_size": [_I64] * 6 + [_INT],
    "gdn_recurrent_fwd": [_P] * 9 + [_I64] * 7 + [_INT] * 3 + [_F, _U, _P, _P, _P],
    "gdn_decode_step": [_P] * 7 + [_I64] * 5 + [_INT] * 4 + [_F, _U, _P, _P, _P],
    "gdn_causal_conv1d_fwd": [_P] * 7 + [_I64] * 5 + [_INT, _INT, _U, _P],
    "gdn_l2norm_fwd": [_P, _P, _I64, _I64, _INT, _F, _P],
    "gdn_rms_norm_gated_fwd": [_P] * 5 + [_I64, _I64, _INT, _F, _INT, _P],
    "gdn_causal_conv1d_bwd": [_P] * 6 + [_I64] * 5 + [_INT, _INT, _U] + [_P] * 5 + [_SZ, _P],
    "gdn_causal_conv1d_bwd_workspace_size": [_I64] * 4,
    "gdn_l2norm_bwd": [_P, _P, _P, _I64, _I64, _INT, _F, _P],
    "gdn_rms_norm_gated_bwd": [_P] * 9 + [_I64, _I64, _INT, _F, _INT, _P, _SZ, _P],
    "gdn_rms_norm_gated_bwd_workspace_size": [_I64, _I64],
    "gdn_qkv_conv_fwd": [_P, _I64, _P, _P, _P, _P, _P, _P] + [_I64] * 6 + [_INT, _INT, _U, _P],
    "gdn_attn_qk_norm_rope_fwd": [_P, _I64, _P, _I64, _P, _P, _INT, _P, _P, _P] + [_I64] * 6 + [_INT, _F, _F, _U, _P],
    "gdn_attn_fwd": [_P, _P, _P, _I64, _P, _I64, _P, _P] + [_I64] * 6 + [_F, _U, _P],
}

RESTYPES = {
    "gdn_last_error": ctypes.c_char_p,
    "gdn_chunk_workspace_size": ctypes.c_size_t,
    "gdn_chunk_gated_norm_workspace_size": ctypes.c_size_t,
    "gdn_chunk_states_size": ctypes.c_size_t,
    "gdn_chunk_fwd_noalloc_max_workspace": ctypes.c_size_t,
    "gdn_chunk_bwd_workspace_size": ctypes.c_size_t,
    "gdn_causal_conv1d_bwd_workspace_size": ctypes.c_size_t,
    "gdn_rms_norm_gated_bwd_workspace_size": ctypes.c_size_t,
}

_lib = None


class GDNError(RuntimeError):
    """A libgdn.so entry point returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argument types declared for every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built. Build it with `python -m sorernn_amd.build` "
            "(hipcc --offload-arch=gfx950); the GDN path has no CPU fallback."
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    ver = lib.gdn_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libgdn.so ABI version {ver} != expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise ``GDNError`` (or ``ValueError``/``NotImplementedError``) on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != GDN_OK:
        msg = lib.gdn_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        if rc == 2:
            raise NotImplementedError(f"{name}: {msg}")
        raise GDNError(f"{name} failed (status {rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported dtype {dt} (float32, bfloat16 or float16)")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def raw_stream(device: torch.device) -> int:
    """The current stream of ``device`` as a raw handle, without building a ``torch.cuda.Stream`` object
    (the per-token decode path's host time)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
