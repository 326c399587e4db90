"""MI355X (gfx950) drop-in for hachiue's logits-to-token sampler.

The host layers (this Python package and the Node-API addon under node/)
call one C ABI, include/hachiue_sampler.h, implemented by hand-written HIP
kernels in csrc/ and built into lib/libhachiue_sampler.so.
"""
from .sampler import (  # noqa: F401
    EXPORTS,
    OPTIONS,
    ROW_GREEDY,
    ROW_REPLAYED,
    ROW_SINGLE,
    ROW_TIES,
    Sampler,
    SamplerError,
    make_configs,
    resolve_config,
    sample_logits,
)
