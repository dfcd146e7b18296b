"""CPU oracle for nano-qwen's GQA attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the timed
CPU baseline.  The product path (``nano_qwen_amd``) never imports it and has no
CPU fallback.
"""

from .attention_oracle import (  # noqa: F401
    rms_norm,
    rope_inv_freq,
    yarn_correction_range,
    yarn_inv_freq,
    rope_tables,
    rotate_half,
    attention,
    attention_path,
    reference_path_sdpa,
    reference_decode_sdpa,
    reference_chunk_sdpa,
    decode_path,
    attention_module_forward,
    OracleKVCache,
)
from .model_oracle import (  # noqa: F401
    swiglu,
    model_forward,
    greedy_reference_protocol,
    greedy_full_recompute,
)
from .ring_oracle import (  # noqa: F401
    ring_attention,
    merge_partials,
    attention_lse,
)
