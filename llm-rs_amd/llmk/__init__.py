"""llmk — MI355X-native batched token sampling for llm-rs (HIP kernels behind a C ABI)."""
from ._lib import LIB_PATH, EXPORTED_SYMBOLS, load  # noqa: F401
from .sampler import (  # noqa: F401
    BatchResult,
    DeviceBatch,
    HipSampler,
    SampleParams,
    SamplerError,
    apply_top_k,
    apply_top_p,
    device_batch_from_params,
    sample,
    sample_batch_static,
    sample_logits,
)
