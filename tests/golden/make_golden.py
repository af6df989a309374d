"""Write the golden vectors of the GDN path under ``tests/golden/`` (run from the repository root).

``python tests/golden/make_golden.py`` regenerates ``gdn_golden.npz``. The vectors come from this
repository's own oracle (``oracle/gdn_oracle.py``) in fp64, not from the reference, whose tests hold
no binary fixtures for this path. Two cases:

- ``c0_*``: BASELINE config 0 exactly (B=1, T=256, H=4, d_k=d_v=64, fp32 inputs from
  ``sorernn_amd.synthetic.config_inputs(0)``, zero initial state, chunk 64) -> ``o`` and the final
  state, computed by the token recurrence (``sore/model/gdn_ref.py:11-22`` order) in fp64;
- ``vl_*``: a small varlen case (3 documents of 37, 64 and 27 tokens, GVA 2, d_k=d_v=64,
  per-document initial states) -> ``o`` and the three final states.

Inputs are stored in fp32 (what the kernels read), outputs in fp64.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import recurrent_gated_delta_rule  # noqa: E402
from sorernn_amd.synthetic import config_inputs, gdn_inputs  # noqa: E402

PATH = os.path.join(HERE, "gdn_golden.npz")
VARLEN_CU = [0, 37, 101, 128]


def varlen_inputs():
    cu = torch.tensor(VARLEN_CU, dtype=torch.long)
    return gdn_inputs(1, VARLEN_CU[-1], 2, 64, V=64, HV=4, dtype=torch.float32, seed=2024, h0=True, cu_seqlens=cu)


def _run(inp):
    d = lambda x: None if x is None else x.double()  # noqa: E731
    return recurrent_gated_delta_rule(d(inp.q), d(inp.k), d(inp.v), d(inp.g), d(inp.beta), inp.scale, d(inp.h0), True,
                                      cu_seqlens=inp.cu_seqlens)


def make() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for tag, inp in (("c0", config_inputs(0)), ("vl", varlen_inputs())):
        o, st = _run(inp)
        for name in ("q", "k", "v", "g", "beta"):
            out[f"{tag}_{name}"] = getattr(inp, name).float().numpy()
        if inp.h0 is not None:
            out[f"{tag}_h0"] = inp.h0.float().numpy()
        if inp.cu_seqlens is not None:
            out[f"{tag}_cu_seqlens"] = inp.cu_seqlens.numpy()
        out[f"{tag}_scale"] = np.array(inp.scale, dtype=np.float64)
        out[f"{tag}_o"] = o.numpy()
        out[f"{tag}_final_state"] = st.numpy()
    return out


if __name__ == "__main__":
    arrays = make()
    np.savez_compressed(PATH, **arrays)
    print(f"wrote {PATH}: " + ", ".join(f"{k}{list(v.shape)}" for k, v in arrays.items()))
