"""MI355X-native (gfx950) fused attention for llmtie-rs: prefill, decode and
KV-cache producers behind the reference's `Gpu` operator interface.

The product is the C-ABI library `libllmtie_hip.so` (include/llmtie_hip.h);
`ttsxabe_amd.gpu.Gpu` is its host-side mirror of `llmtie_cuda::Gpu`.
"""
from .build import LIB  # noqa: F401

__version__ = "0.1.0"


def __getattr__(name):
    # The torch-facing host mirror is imported lazily so that building the
    # library does not need torch.
    if name in ("Gpu", "DecodeScratch", "Q8", "KvCacheQ8", "gpu"):
        from . import gpu as _g
        return _g if name == "gpu" else getattr(_g, name)
    raise AttributeError(name)
