"""Full-size GPU parity against the committed oracle fixtures (tests/golden/*.npz).

The fixtures hold the oracle's outputs for the seeded synthetic inputs of
``mirror_sd_amd.synth`` at the real shapes of the 8B-class draft (5 layers, H4096,
block 16, context 2048) and the 27B-class headline draft (5 layers, H5120, block 32,
context 4096), so the HIP path is checked at full size without running the oracle on
the GPU host.  Tolerances: final hidden cosine >= 0.9995 and max-abs <= 2e-2 (fp16);
argmax identical on every row except where the oracle itself is undecided: its runs that
differ in accumulation only (fp32, fp64, and fp32 with every reduction summed over 2, 4 or
8 ordered k-ranges, all stored in the fixture) do not all agree, and the GPU picked one of
their ids -- at most the committed number of such rows per fixture -- or the row is the one
listed with its id in parity_util.KNOWN_UNBACKED (check_argmax states the rule and prints
the counts); GPU logits at the oracle's top-2 indices within LOGIT_TOL of the oracle's
values.
"""

import os

import numpy as np
import pytest

from golden.make_golden import input_digests
from mirror_sd_amd import synth
from mirror_sd_amd.config import workload
from parity_util import (assert_close_fp16, check_argmax, device_errors, oracle_alt_runs,
                         torch_tensors)

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LOGIT_TOL = 2e-2


def load(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def test_single_layer_matches_golden():
    """1 layer, H2560, 32/8 heads, FFN 9728, block 16, context 64, fused inputs."""
    from mirror_sd_amd.dflash import DFlashDraftModel
    g = load("qwen3_4b_layer")
    wl = workload("qwen3_4b_layer")
    t = synth.make_weights_numpy(wl.cfg, seed=0, with_vocab=False, with_fc=False)
    inp = synth.make_inputs_numpy(wl.cfg, wl.block, wl.ctx, seed=0, fused_context=True)
    m = DFlashDraftModel(wl.cfg, max_ctx=wl.ctx, n_target_feat=0)
    m.load_weights(torch_tensors(t, "cuda"))
    m.make_cache(0, 0)
    m._ingest(torch.from_numpy(inp["context"]), fused=True)
    h, pre, _, _ = m._draft(noise=torch.from_numpy(inp["noise"]), want_prenorm=True)
    torch.cuda.synchronize()
    assert_close_fp16(pre.float().cpu().numpy(), g["prenorm"], what="layer output")
    assert_close_fp16(h.float().cpu().numpy(), g["hidden"], what="final-normed output")
    m.close()


@pytest.mark.parametrize("name", ["qwen3_8b_draft", "dflash_27b"])
def test_full_draft_matches_golden(name):
    from mirror_sd_amd.dflash import DFlashDraftModel
    g = load(name)
    wl = workload(name)
    print(f"case {name}: generating inputs", flush=True)
    t = synth.make_weights_numpy(wl.cfg, seed=0)
    inp = synth.make_inputs_numpy(wl.cfg, wl.block, wl.ctx, seed=0)
    assert input_digests(t, inp) == dict(zip(g["digest_names"].tolist(),
                                             g["digest_values"].tolist()))
    m = DFlashDraftModel(wl.cfg, max_ctx=wl.ctx)
    m.load_weights(torch_tensors(t, "cuda"))
    del t
    torch.cuda.empty_cache()
    print(f"case {name}: drafting", flush=True)
    ids, logits, h = m.draft(torch.from_numpy(inp["ids"]), torch.from_numpy(inp["target_hidden"]),
                             return_logits=True, return_hidden=True)
    torch.cuda.synchronize()
    assert_close_fp16(h.float().cpu().numpy(), g["hidden"], what=f"{name} final hidden")
    lg = logits.cpu().numpy()
    ids = ids.cpu().numpy()
    check_argmax(ids, lg, g["ids"], oracle_alt_runs(g), name, g["top2_idx"], g["top2_val"], LOGIT_TOL)
    # the lm_head hands half tiles out at run time from self-resetting counters: later
    # launches on the same inputs give the same bits, and no queue wait gave up
    for rep in range(2):
        ids2, logits2, _ = m.draft(torch.from_numpy(inp["ids"]),
                                   torch.from_numpy(inp["target_hidden"]), return_logits=True,
                                   return_hidden=True)
        ids3 = m.draft(torch.from_numpy(inp["ids"]), torch.from_numpy(inp["target_hidden"]))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids2.cpu().numpy(), ids)
        np.testing.assert_array_equal(logits2.cpu().numpy(), lg)
        np.testing.assert_array_equal(ids3.cpu().numpy(), ids)
    assert device_errors(m) == 0
    m.close()


# ---------------------------------------------------------------------------
# Context sweep: the 27B-class draft at contexts 64 .. 32768 (context 4096 is the case
# above).  One model (seed-0 weights, cache for 32768 rows) drafts against each context.
# ---------------------------------------------------------------------------

SWEEP = (64, 2048, 16384, 32768)


@pytest.fixture(scope="module")
def sweep_model():
    from mirror_sd_amd.dflash import DFlashDraftModel
    wl = workload("dflash_27b_ctx32768")
    print("context sweep: generating weights", flush=True)
    t = synth.make_weights_numpy(wl.cfg, seed=0)
    m = DFlashDraftModel(wl.cfg, max_ctx=max(SWEEP))
    m.load_weights(torch_tensors(t, "cuda"))
    digests = input_digests(t, {})
    del t
    torch.cuda.empty_cache()
    yield m, digests
    m.close()


def _check_against(g, name, ids, logits, h):
    assert_close_fp16(h.float().cpu().numpy(), g["hidden"], what=f"{name} final hidden")
    check_argmax(ids.cpu().numpy(), logits.cpu().numpy(), g["ids"], oracle_alt_runs(g), name,
                 g["top2_idx"], g["top2_val"], LOGIT_TOL)


@pytest.mark.parametrize("ctx", SWEEP)
def test_context_sweep_matches_golden(sweep_model, ctx):
    m, wdig = sweep_model
    name = f"dflash_27b_ctx{ctx}"
    g = load(name)
    wl = workload(name)
    print(f"case {name}: generating inputs", flush=True)
    inp = synth.make_inputs_numpy(wl.cfg, wl.block, wl.ctx, seed=0)
    want = dict(zip(g["digest_names"].tolist(), g["digest_values"].tolist()))
    got = dict(wdig)
    got.update(input_digests({}, inp))
    assert got == want
    print(f"case {name}: drafting", flush=True)
    th = torch.from_numpy(inp["target_hidden"]).cuda()
    ids, logits, h = m.draft(torch.from_numpy(inp["ids"]), th, return_logits=True,
                             return_hidden=True)
    torch.cuda.synchronize()
    _check_against(g, name, ids, logits, h)
    if ctx == max(SWEEP):
        # the same context ingested in three uneven calls (a 31-row one among them)
        from mirror_sd_amd import _lib
        _lib.check(m._L.dfl_cache_reset(m._ctx), "dfl_cache_reset")
        m._gen += 1
        for a, b in ((0, 5000), (5000, 5031), (5031, ctx)):
            m._ingest(th[a:b])
        h2, _, lg2, ids2 = m._draft(ids=torch.from_numpy(inp["ids"]), want_logits=True,
                                    want_ids=True)
        torch.cuda.synchronize()
        _check_against(g, name + " (chunked ingest)", ids2, lg2, h2)


def test_decode_loop_matches_golden():
    """The 27B-class draft in a decode loop: 4096 context rows ingested at once (library
    GEMMs), then 1, 16 and 32 more rows per step (the stream-K per-step ingest), a block of
    32 drafted after each step against the oracle's single pass over the same prefix."""
    from golden.make_golden import STEADY_BASE, STEADY_STEPS
    from mirror_sd_amd import _lib
    from mirror_sd_amd.dflash import DFlashDraftModel
    name = "dflash_27b_steady"
    g = load(name)
    wl = workload("dflash_27b")
    total = STEADY_BASE + sum(STEADY_STEPS)
    print(f"case {name}: generating inputs", flush=True)
    t = synth.make_weights_numpy(wl.cfg, seed=0)
    inp = synth.make_inputs_numpy(wl.cfg, wl.block, total, seed=0)
    assert input_digests(t, inp) == dict(zip(g["digest_names"].tolist(),
                                             g["digest_values"].tolist()))
    m = DFlashDraftModel(wl.cfg, max_ctx=total)
    m.load_weights(torch_tensors(t, "cuda"))
    del t
    torch.cuda.empty_cache()
    th = torch.from_numpy(inp["target_hidden"]).cuda()
    ids = torch.from_numpy(inp["ids"])
    _lib.check(m._L.dfl_cache_reset(m._ctx), "dfl_cache_reset")
    m._gen += 1
    m._ingest(th[:STEADY_BASE])
    n = STEADY_BASE
    for i, k in enumerate(STEADY_STEPS):
        print(f"case {name}: step {i}, {k} new rows", flush=True)
        m._ingest(th[n:n + k])
        n += k
        h, _, lg, idg = m._draft(ids=ids, want_logits=True, want_ids=True)
        torch.cuda.synchronize()
        assert_close_fp16(h.float().cpu().numpy(), g[f"s{i}_hidden"], what=f"{name} step {i} hidden")
        check_argmax(idg.cpu().numpy(), lg.cpu().numpy(), g[f"s{i}_ids"], oracle_alt_runs(g, f"s{i}_"),
                     f"{name} step {i} ({n} context rows)", g[f"s{i}_top2_idx"],
                     g[f"s{i}_top2_val"], LOGIT_TOL)
    assert device_errors(m) == 0
    m.close()
