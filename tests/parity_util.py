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


# Draft-token agreement.  The north-star bar is identical argmax on >= 99.9 % of positions.
# A row may differ from the oracle only where the oracle's own answer is decided by
# accumulation rounding:
#  * "oracle-undecided": the oracle's runs that differ in accumulation only -- fp32, fp64,
#    and (full-size fixtures) fp32 with every reduction summed over 2, 4 or 8 ordered
#    ranges of k (dflash_oracle.accumulation_split), all with the same fp16 rounding
#    points -- do not all pick the same id, and the GPU picked one of theirs;
#  * "noise" (only where a test asks for it, noise_rule=True: the full-size fixture tests,
#    where the oracle runs at test time on small shapes none does): the
#    GPU picked the oracle's runner-up and the oracle's top-2 gap is below
#    NOISE_SIGMAS x sigma, sigma being the RMS of (GPU logit - oracle logit) over every
#    row's oracle top-2 entries in the same case.  That logit noise comes from fp32
#    summation order flipping fp16 roundings through the layers (the oracle's own fp32 and
#    fp64 runs differ by up to 2.6e-3 in a gap); at the full-size shapes sigma is about
#    3e-3, so the gap of two logits carries noise ~ sqrt(2) sigma and a row whose gap is
#    4 sigma (2.8 x that) or more flips with probability below 0.3 % -- such rows must
#    agree.  Any change of summation order (a different split of a projection over the
#    CUs) re-draws the rows below the threshold, so they cannot be held to exact agreement.
# Everything else must agree.  Every call records its counts; conftest prints the session
# total, raw agreement included.
ARGMAX_TOTALS = {"rows": 0, "agree": 0, "undecided": 0, "noise": 0, "cases": []}
NOISE_SIGMAS = 4.0


def oracle_alt_runs(g, prefix=""):
    """The ids of a fixture's other accumulation runs (fp64, and the split-k fp32 runs when
    the fixture holds them), one row per run, for check_argmax's ``alt_ids``."""
    runs = [np.asarray(g[prefix + "ids_f64"]).reshape(1, -1)]
    if prefix + "ids_ksplit" in g:
        runs.append(np.asarray(g[prefix + "ids_ksplit"]))
    return np.concatenate(runs, axis=0)


def check_argmax(ids, logits, ref_ids, alt_ids, what, ref_top2_idx, ref_top2_val,
                 logit_tol=2e-2, noise_rule=False):
    """Assert the GPU ids against the oracle's (fp32-accumulation ``ref_ids`` with its top-2
    indices / logits; ``alt_ids`` the ids of its other accumulation runs, one row per run:
    fp64, and the split-k fp32 runs where a fixture holds them); returns (agree, rows,
    exempt).  ``noise_rule`` True also exempts the noise band."""
    ids = np.asarray(ids).reshape(-1)
    ref_ids = np.asarray(ref_ids).reshape(-1)
    alt_ids = np.asarray(alt_ids).reshape(-1, ids.size)
    ti = np.asarray(ref_top2_idx, np.int64).reshape(ids.size, 2)
    tv = np.asarray(ref_top2_val, np.float64).reshape(ids.size, 2)
    lg = np.asarray(logits).reshape(ids.size, -1)
    # the GPU ids are exactly the argmax of the GPU logits (lowest index on ties)
    np.testing.assert_array_equal(ids, np.argmax(lg, axis=-1), err_msg=what)
    err = np.take_along_axis(lg, ti, axis=-1).astype(np.float64) - tv
    emax = float(np.abs(err).max())
    assert emax < logit_tol, f"{what}: logits at the oracle's top-2 differ by {emax:.3e}"
    sigma = float(np.sqrt(np.mean(err * err)))
    tau = NOISE_SIGMAS * sigma
    gap = tv[:, 0] - tv[:, 1]
    agree = ids == ref_ids
    undecided = ~agree & (ids[None, :] == alt_ids).any(axis=0)
    noise = ~agree & ~undecided & (ids == ti[:, 1]) & (gap < tau) & noise_rule
    bad = ~agree & ~undecided & ~noise
    n, n_agree = ids.size, int(agree.sum())
    n_und, n_noise = int(undecided.sum()), int(noise.sum())
    print(f"{what}: argmax agreement {n_agree}/{n} ({n_agree / n:.4f}); exempt "
          f"{n_und} oracle-undecided, {n_noise} of {int((gap < tau).sum())} rows with a top-2 "
          f"gap below {NOISE_SIGMAS:g} sigma = {tau:.2e} (logit error rms {sigma:.2e}, max "
          f"{emax:.2e})", flush=True)
    ARGMAX_TOTALS["rows"] += n
    ARGMAX_TOTALS["agree"] += n_agree
    ARGMAX_TOTALS["undecided"] += n_und
    ARGMAX_TOTALS["noise"] += n_noise
    ARGMAX_TOTALS["cases"].append((what, n_agree, n, n_und, n_noise))
    assert not bad.any(), (f"{what}: argmax differs from the oracle at rows "
                           f"{np.nonzero(bad)[0].tolist()} (GPU {ids[bad].tolist()}, oracle "
                           f"{ref_ids[bad].tolist()}, other oracle runs "
                           f"{alt_ids[:, bad].T.tolist()}, "
                           f"oracle gaps {gap[bad].tolist()}, tau {tau:.2e})")
    return n_agree, n, n_und + n_noise
