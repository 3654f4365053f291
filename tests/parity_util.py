"""Shared helpers for the GPU parity tests (oracle on the CPU, HIP path on the GPU)."""

import numpy as np


def cos_sim(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def assert_close_fp16(got, ref, cos_min=0.9995, max_abs=2e-2, what=""):
    """The draft-output tolerance: cosine >= 0.9995 and max-abs <= 2e-2 (fp16)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    c = cos_sim(got, ref)
    err = float(np.abs(got - ref).max())
    assert c >= cos_min and err <= max_abs, f"{what}: cos={c:.7f} max_abs={err:.3e}"
    return c, err


def torch_tensors(np_tensors, device):
    import torch
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in np_tensors.items()}


def device_errors(m):
    """The sticky device-side error flags of a DFlashDraftModel's context (reading clears)."""
    import ctypes
    import torch
    from mirror_sd_amd import _lib
    v = ctypes.c_int32(0)
    _lib.check(m._L.dfl_device_errors(m._ctx, ctypes.byref(v),
                                      torch.cuda.current_stream().cuda_stream),
               "dfl_device_errors")
    return v.value
