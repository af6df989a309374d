"""MI355X-native (gfx950) Gated DeltaNet token-mixing path for soreRNN.

A drop-in for FLA's ``chunk_gated_delta_rule`` / ``fused_recurrent_gated_delta_rule`` and the conv
and gated-norm modules used by ``sore/model/gdn.py``: Python host code calls the C ABI of
``libgdn.so`` (``include/gdn.h``), which launches hand-written HIP kernels built for gfx950.
"""
from sorernn_amd.ops import (  # noqa: F401
    causal_conv1d,
    chunk_gated_delta_rule,
    chunk_gated_delta_rule_gated_norm,
    fused_recurrent_gated_delta_rule,
    gated_delta_decode_step,
    l2norm,
    rms_norm_gated,
)
from sorernn_amd.range_guard import check_chunk_range, range_guard, set_range_guard  # noqa: F401

__version__ = "0.1.0"
