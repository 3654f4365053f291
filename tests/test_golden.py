"""The committed golden fixtures (tests/golden/*.npz, written by make_golden.py) against
the current input recipe and the oracle, on the CPU.

* every fixture's input digests match what ``mirror_sd_amd.synth`` generates now, so a
  GPU test comparing against a fixture runs on the inputs the fixture was made from;
* the oracle reproduces the single-layer fixture exactly (fp64 accumulation with fp16
  rounding points is deterministic), which pins the oracle against regressions.
"""

import os

import numpy as np
import pytest

from golden.make_golden import case_layer, input_digests
from mirror_sd_amd import synth
from mirror_sd_amd.config import workload

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def stored_digests(g):
    return dict(zip(g["digest_names"].tolist(), g["digest_values"].tolist()))


@pytest.mark.parametrize("name", ["qwen3_8b_draft", "dflash_27b"])
def test_full_fixture_inputs_match_recipe(name):
    wl = workload(name)
    t = synth.make_weights_numpy(wl.cfg, seed=0)
    inp = synth.make_inputs_numpy(wl.cfg, wl.block, wl.ctx, seed=0)
    assert input_digests(t, inp) == stored_digests(load(name))


def test_layer_fixture_reproduced_by_oracle():
    g = load("qwen3_4b_layer")
    out, dig = case_layer("qwen3_4b_layer")
    assert dig == stored_digests(g)
    np.testing.assert_array_equal(out["hidden"], g["hidden"])
    np.testing.assert_array_equal(out["prenorm"], g["prenorm"])


@pytest.mark.parametrize("name", ["qwen3_8b_draft", "dflash_27b"])
def test_full_fixture_consistent(name):
    """ids are the fixture's own top-1; rows are unit-rms after the final norm."""
    g = load(name)
    wl = workload(name)
    assert g["ids"].shape == (wl.block,) and g["hidden"].shape == (wl.block, wl.cfg.hidden_size)
    np.testing.assert_array_equal(g["ids"], g["top2_idx"][:, 0])
    assert np.all(g["top2_val"][:, 0] >= g["top2_val"][:, 1])
    rms = np.sqrt((g["hidden"].astype(np.float64) ** 2).mean(-1))
    np.testing.assert_allclose(rms, 1.0, atol=5e-3)   # norm gains are 1


def test_batch_fixture_inputs_match_recipe():
    name = "llama8b_batch"
    wl = workload(name)
    t = synth.make_weights_numpy(wl.cfg, seed=0)
    inps = synth.make_batch_inputs_numpy(wl.cfg, wl.block, wl.seq_ctx, seed=0)
    dig = input_digests(t, {f"{k}.s{i}": v for i, inp in enumerate(inps) for k, v in inp.items()})
    g = load(name)
    assert dig == stored_digests(g)
    assert g["ids"].shape == (wl.block * len(wl.seq_ctx),)
    np.testing.assert_array_equal(g["ids"], g["top2_idx"][:, 0])
