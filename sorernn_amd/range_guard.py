"""Range guard of the chunked forward: reports non-finite outputs.

The chunk forward (``gdn_chunk.hip``) feeds the state S, X, Delta, T - I and scale * P to the
matrix cores as fp16, whose largest finite value is 65504; FLA's kernels use bf16 operands, which
keep fp32's exponent range. A workgroup of the chunk kernel whose fp16 operands overflow (it stored
an inf or NaN in ``o`` or the final state) computes its columns again by the fp32 token-by-token
recurrence before it exits, so finite inputs whose fp32 results are finite give finite outputs.
The kernel then sets a flag word (``gdn_set_range_flag`` in ``include/gdn.h``) only when that
recomputation is non-finite too: non-finite inputs, for which FLA returns non-finite outputs as
well. (The cooperative prefill, selected with ``SORERNN_PREFILL=coop``, has no such recomputation
and sets the flag on its own non-finite outputs.) This module keeps one pinned host word per device,
registered with the library on the first chunk call on that device, and decides what a set flag
does:

- ``"warn"`` (the default): no synchronisation. A flag that earlier calls set is cleared and
  reported with a ``RuntimeWarning`` by the next ``chunk_gated_delta_rule`` call on that device,
  or by ``check_chunk_range()``.
- ``"raise"``: every call waits for its stream and raises ``FloatingPointError`` if it set the flag.
- ``"fallback"``: every call waits for its stream; a call that set the flag is computed again by
  the fp32 recurrent kernel (the same recurrence token by token, no fp16 operands), with a
  warning the first time. A call that needs a backward cannot fall back (the backward reads the
  chunk forward's saved states) and raises instead.
- ``"off"``: no flag, no check.

``SORERNN_RANGE_GUARD`` sets the initial mode.
"""
from __future__ import annotations

import os
import warnings

import numpy as np
import torch

from sorernn_amd import _lib

MODES = ("warn", "raise", "fallback", "off")

_mode = os.environ.get("SORERNN_RANGE_GUARD", "warn")
if _mode not in MODES:
    raise ValueError(f"SORERNN_RANGE_GUARD={_mode!r}: expected one of {MODES}")
_words: dict[int, tuple[torch.Tensor, np.ndarray]] = {}
# Flag words unregistered by set_range_guard("off"). Kernels still in flight, and graphs captured
# while a word was registered, keep its address, so a word is never freed before the process ends.
_retired: list[torch.Tensor] = []
_fallback_noted = False

_EARLIER = ("chunk_gated_delta_rule: an earlier chunked forward on cuda:{dev} stored inf or NaN outputs (non-finite "
            "inputs, or an fp16 operand of the chunk kernel past 65504 that its fp32 recomputation did not bring "
            "back into range). Set sorernn_amd.set_range_guard('fallback') to recompute such calls with the fp32 "
            "recurrent kernel, or 'raise' to stop at the call.")


def set_range_guard(mode: str) -> None:
    """Select what a non-finite chunk output does: ``"warn"``, ``"raise"``, ``"fallback"`` or ``"off"``."""
    global _mode
    if mode not in MODES:
        raise ValueError(f"set_range_guard: mode must be one of {MODES}, got {mode!r}")
    _mode = mode
    if mode == "off":
        for dev in list(_words):
            _lib.call("gdn_set_range_flag", dev, None)
            # kept alive: launches in flight and captured graphs may still store into it
            _retired.append(_words.pop(dev)[0])


def range_guard() -> str:
    """The current mode."""
    return _mode


def _device_index(device: torch.device | int | None) -> int:
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    return device.index if device.index is not None else torch.cuda.current_device()


def _word(dev: int) -> np.ndarray:
    w = _words.get(dev)
    if w is None:
        t = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        _lib.call("gdn_set_range_flag", dev, t.data_ptr())
        w = _words[dev] = (t, t.numpy())
    return w[1]


def before_call(device: torch.device) -> np.ndarray | None:
    """Before a chunk launch (eager calls): the device's flag word, after reporting and clearing a
    flag left by earlier calls. None when the guard is off."""
    if _mode == "off":
        return None
    dev = _device_index(device)
    word = _word(dev)
    if word[0]:
        word[0] = 0
        warnings.warn(_EARLIER.format(dev=dev), RuntimeWarning, stacklevel=4)
    return word


def call_overflowed(word: np.ndarray | None, device: torch.device) -> bool:
    """After a chunk launch in the "raise" and "fallback" modes: wait for the call's stream and
    return True (clearing the word) when the call set the flag. False in the other modes, and during
    HIP graph capture (a synchronisation would invalidate the capture): a captured call is then
    reported as in "warn" mode, by the next eager call or ``check_chunk_range()``.

    The word is per device, not per call or stream: a flag that a call on another stream of the
    device set while this one ran is reported here as well."""
    if word is None or _mode not in ("raise", "fallback"):
        return False
    if torch.cuda.is_current_stream_capturing():
        return False
    torch.cuda.current_stream(device).synchronize()
    if not word[0]:
        return False
    word[0] = 0
    return True


def note_fallback(name: str) -> None:
    global _fallback_noted
    if not _fallback_noted:
        _fallback_noted = True
        warnings.warn(f"{name}: a chunked forward overflowed its fp16 operands (or saw non-finite inputs); "
                      "recomputed with the fp32 recurrent kernel (reported once per process)",
                      RuntimeWarning, stacklevel=4)


def check_chunk_range(device: torch.device | int | None = None, clear: bool = True) -> bool:
    """Wait for the device and return whether a chunked forward on it stored an inf or NaN since the
    flag was last cleared. The flag is cleared unless ``clear=False``. Always False when the guard is
    off or no chunk call has run on the device."""
    dev = _device_index(device)
    w = _words.get(dev)
    if w is None:
        return False
    torch.cuda.synchronize(dev)
    hit = bool(w[1][0])
    if hit and clear:
        w[1][0] = 0
    return hit
