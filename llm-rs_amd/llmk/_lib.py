"""ctypes binding of the C ABI declared in include/llmk_sampler.h.

The shared library is built in-tree by __graft_entry__.build() (or
`make -C llm-rs_amd`) into llm-rs_amd/llmk/libllmk_sampler.so.  There is no
fallback: if the library is missing, loading raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libllmk_sampler.so")

LLMK_OK = 0
LLMK_ERR_INVALID_ARGUMENT = -1
LLMK_ERR_EMPTY_LOGITS = -2
LLMK_ERR_CAPACITY = -3
LLMK_ERR_HIP = -4
LLMK_ERR_ALIGNMENT = -5
LLMK_ERR_UNSUPPORTED = -6
LLMK_INVALID_TOKEN = 0xFFFFFFFF
LLMK_STATUS_INVALID_PARAMS = 0x1
LLMK_STATUS_HISTORY_OVERFLOW = 0x2
LLMK_STATUS_SLOT_TIMEOUT = 0x4
LLMK_STATUS_HISTORY_FULL = 0x8
LLMK_STATUS_NAN_LOGITS = 0x10
LLMK_F32 = 0
LLMK_BF16 = 1
LLMK_F16 = 2

# Every symbol include/llmk_sampler.h declares (checked by the CPU tests).
EXPORTED_SYMBOLS = (
    "llmk_sampler_create",
    "llmk_sample_batch",
    "llmk_sampler_status",
    "llmk_sampler_destroy",
    "llmk_last_error",
    "llmk_apply_top_k",
    "llmk_apply_top_p",
    "llmk_apply_logit_bias",
    "llmk_history_append",
    "llmk_history_count_append",
    "llmk_sample_batch_static",
    "llmk_verify_batch",
)


class SampleBatchArgs(ctypes.Structure):
    """Mirror of llmk_sample_batch_args (include/llmk_sampler.h)."""

    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32),
        ("row_stride", ctypes.c_uint64),
        ("temperature", ctypes.c_void_p),
        ("top_k", ctypes.c_void_p),
        ("top_p", ctypes.c_void_p),
        ("min_p", ctypes.c_void_p),
        ("repetition_penalty", ctypes.c_void_p),
        ("presence_penalty", ctypes.c_void_p),
        ("frequency_penalty", ctypes.c_void_p),
        ("hist_offsets", ctypes.c_void_p),
        ("hist_tokens", ctypes.c_void_p),
        ("allow_mask", ctypes.c_void_p),
        ("mask_words_per_row", ctypes.c_uint32),
        ("uniforms", ctypes.c_void_p),
        ("out_tokens", ctypes.c_void_p),
        ("out_ids", ctypes.c_void_p),
        ("out_probs", ctypes.c_void_p),
        ("out_cap", ctypes.c_uint32),
        ("out_count", ctypes.c_void_p),
        ("hist_lengths", ctypes.c_void_p),
        ("softcap", ctypes.c_float),
        ("hist_counts", ctypes.c_void_p),
    ]


_lib = None


def load():
    """Load libllmk_sampler.so (raises OSError if it was never built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(the sampler has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    vp = ctypes.c_void_p
    lib.llmk_sampler_create.argtypes = [ctypes.POINTER(vp), ctypes.c_int,
                                        ctypes.c_uint32, ctypes.c_uint32]
    lib.llmk_sampler_create.restype = ctypes.c_int
    lib.llmk_sample_batch.argtypes = [vp, ctypes.POINTER(SampleBatchArgs), vp]
    lib.llmk_sample_batch.restype = ctypes.c_int
    lib.llmk_sample_batch_static.argtypes = [ctypes.POINTER(SampleBatchArgs), vp, vp]
    lib.llmk_sample_batch_static.restype = ctypes.c_int
    lib.llmk_sampler_status.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_uint32)]
    lib.llmk_sampler_status.restype = ctypes.c_int
    lib.llmk_sampler_destroy.argtypes = [vp]
    lib.llmk_sampler_destroy.restype = None
    for fn, par in (("llmk_apply_top_k", vp), ("llmk_apply_top_p", vp)):
        getattr(lib, fn).argtypes = [vp, vp, ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.c_uint64, par, vp]
        getattr(lib, fn).restype = ctypes.c_int
    lib.llmk_apply_logit_bias.argtypes = [vp, vp, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_uint64, vp, vp, vp, vp]
    lib.llmk_apply_logit_bias.restype = ctypes.c_int
    lib.llmk_history_append.argtypes = [vp, ctypes.c_uint32, vp, vp, vp, ctypes.c_uint32, vp, vp]
    lib.llmk_history_append.restype = ctypes.c_int
    lib.llmk_history_count_append.argtypes = [vp, ctypes.c_uint32, vp, vp, vp, vp,
                                              ctypes.c_uint32, vp, vp]
    lib.llmk_history_count_append.restype = ctypes.c_int
    u32, u64 = ctypes.c_uint32, ctypes.c_uint64
    lib.llmk_verify_batch.argtypes = [vp, u32, u32, vp, vp, u32, vp, vp, vp, u64, vp, vp, vp, vp,
                                      vp]
    lib.llmk_verify_batch.restype = ctypes.c_int
    lib.llmk_last_error.argtypes = []
    lib.llmk_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def last_error():
    return load().llmk_last_error().decode()
