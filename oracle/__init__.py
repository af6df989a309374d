"""CPU oracle for the Gated DeltaNet token-mixing path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
this package, and only as the checker or the timed CPU baseline. The product path
(``sorernn_amd``) never imports it and has no CPU fallback.
"""
from oracle.gdn_oracle import (  # noqa: F401
    causal_conv1d_silu,
    causal_conv1d_varlen,
    chunk_gated_delta_rule_bwd_ref,
    chunk_gated_delta_rule_ref,
    conv_state_from_sequence,
    decode_step_ref,
    doc_ids_from_cu_seqlens,
    gate_and_beta,
    gva_expand,
    l2norm,
    matrix_transition_rule,
    naive_gated_delta_rule,
    positions_from_cu_seqlens,
    recurrent_gated_delta_rule,
    rms_norm,
    rms_norm_gated,
)
