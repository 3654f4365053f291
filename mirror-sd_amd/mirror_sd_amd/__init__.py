"""MI355X-native DFlash draft forward (W8A16) for mirror-sd.

``DFlashDraftModel`` / ``DFlashConfig`` / ``DFlashKVCache`` mirror mirror_sd/dflash.py;
the compute runs in libdflash_hip.so (HIP kernels for gfx950, C ABI in
include/dflash_hip.h).
"""

from .config import DFlashConfig, Workload, build_target_layer_ids, extract_context_feature, workload

__all__ = ["DFlashConfig", "DFlashDraftModel", "DFlashKVCache", "Workload",
           "build_target_layer_ids", "extract_context_feature", "workload", "sample"]


def __getattr__(name):
    # the model classes load the shared library lazily (first use)
    if name in ("DFlashDraftModel", "DFlashKVCache", "sample"):
        from . import dflash
        return getattr(dflash, name)
    raise AttributeError(name)
