"""Batched drafting (several independent sequences, ragged contexts) on the GPU.

The reference drafts one sequence at a time; a batched block must equal running each
sequence through the single-sequence forward.  Checked against the oracle per sequence
(small shapes, oracle at test time) and, at the 8 x 32-row LLaMA-8B-class shape with
contexts [4146, 4443, 6312, 7812, 779, 1619, 6833, 7798], against the committed fixture.
Tolerances as for the single-sequence draft: hidden cosine >= 0.9995 and max-abs <= 2e-2,
argmax identical except where the oracle's accumulation runs disagree
(parity_util.check_argmax).
"""

import os

import numpy as np
import pytest

from golden.make_golden import input_digests
from mirror_sd_amd import synth
from mirror_sd_amd.config import workload
from oracle import dflash_oracle as O
from parity_util import assert_close_fp16, check_argmax, oracle_alt_runs, torch_tensors

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LOGIT_TOL = 2e-2


def _oracle_both(W, inp):
    """The oracle's fp32-accumulation run (reference ids, logits) and its fp64 run's ids."""
    h, lg, ids = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True, dtype=np.float32)
    _, _, ids64 = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True)
    ti = np.argsort(-lg, axis=-1, kind="stable")[:, :2]
    return h, ids, ids64, ti, np.take_along_axis(lg, ti, -1)


@pytest.mark.parametrize("seq_ctx,B", [((24, 5, 17), 8),                       # 24 rows
                                       ((7, 30, 11, 2, 19, 25, 4, 13), 16),   # 128 rows
                                       ((9, 3, 28, 14, 6, 21), 32),           # 192 rows
                                       ((5, 9, 2, 30, 12, 7, 1, 18, 22, 3), 8)])  # 80 rows
def test_batch_small_matches_oracle_and_single_sequence(seq_ctx, B):
    """Stacked rows below one m-tile (stream-K GEMMs throughout), and 80, 128 and 192 rows
    (tile GEMMs with fused RESID / SWIGLU / ARGMAX epilogues; 80 rows leave a partial
    m-tile whose rows the epilogues must skip); 10 sequences take two rope / attention
    launches (8 + 2)."""
    from mirror_sd_amd.dflash import DFlashDraftModel
    wl = workload("tiny")
    cfg = wl.cfg
    t = synth.make_weights_numpy(cfg, seed=3)
    inps = synth.make_batch_inputs_numpy(cfg, B, seq_ctx, seed=3)
    W = O.OracleWeights(cfg, t)
    m = DFlashDraftModel(cfg, max_ctx=max(seq_ctx), max_block=B, max_seqs=len(seq_ctx))
    m.load_weights(torch_tensors(t, "cuda"))
    for i, inp in enumerate(inps):
        m.ingest_seq(i, torch.from_numpy(inp["target_hidden"]))
    ids_b = np.stack([inp["ids"] for inp in inps])
    ids, logits, h = m.draft_batch(ids=torch.from_numpy(ids_b), return_logits=True,
                                   return_hidden=True)
    torch.cuda.synchronize()
    ids, logits, h = ids.cpu().numpy(), logits.cpu().numpy(), h.float().cpu().numpy()
    refs = [_oracle_both(W, inp) for inp in inps]
    for i, (h_ref, ids_ref, ids64, ti, tv) in enumerate(refs):
        assert_close_fp16(h[i], h_ref, what=f"sequence {i} hidden")
        check_argmax(ids[i], logits[i], ids_ref, ids64, f"batch {seq_ctx} sequence {i}", ti, tv,
                     LOGIT_TOL)
    # the same sequences drafted one at a time through the single-sequence entry point
    # (stream-K GEMMs; the stacked path above may use tile GEMMs, so the two agree to
    # fp32 summation order: hidden within 1e-5 of cosine, ids as against the oracle)
    for i, inp in enumerate(inps):
        m.select_seq(i)
        one = torch.empty(B, dtype=torch.int32, device="cuda")
        hh = torch.empty((B, cfg.hidden_size), dtype=torch.float16, device="cuda")
        lg1 = torch.empty((B, cfg.vocab_size), dtype=torch.float32, device="cuda")
        from mirror_sd_amd import _lib
        idt = torch.from_numpy(inp["ids"]).cuda()
        _lib.check(m._L.dfl_draft_block(m._ctx, None, idt.data_ptr(), B, hh.data_ptr(), None,
                                        lg1.data_ptr(), one.data_ptr(), _lib.stream_handle()),
                   "dfl_draft_block")
        torch.cuda.synchronize()
        _, ids_ref, ids64, ti, tv = refs[i]
        check_argmax(one.cpu().numpy(), lg1.cpu().numpy(), ids_ref, ids64,
                     f"batch {seq_ctx} sequence {i} single", ti, tv, LOGIT_TOL)
        assert_close_fp16(hh.float().cpu().numpy(), h[i], cos_min=0.99999, max_abs=4e-3,
                          what=f"sequence {i} batched vs single")
    m.select_seq(0)
    m.close()


@pytest.mark.parametrize("seq_ctx,B", [((40, 130, 75), 29),      # 87 rows: partial m-tile
                                       ((33, 100, 64, 9), 32)])  # 128 rows
def test_batch_split_k_matches_oracle(seq_ctx, B):
    """H1024 / 8:2 heads / FFN 4096 at 87 and 128 stacked rows: the tile GEMM splits o and
    down over k (fp32 planes summed in order by the reduce kernel with the RESID epilogue),
    against the oracle per sequence."""
    from mirror_sd_amd.config import _draft_cfg
    from mirror_sd_amd.dflash import DFlashDraftModel
    cfg = _draft_cfg(1024, 8, 2, 4096, 2, vocab=4096, block=B)
    t = synth.make_weights_numpy(cfg, seed=4)
    inps = synth.make_batch_inputs_numpy(cfg, B, seq_ctx, seed=4)
    W = O.OracleWeights(cfg, t)
    m = DFlashDraftModel(cfg, max_ctx=max(seq_ctx), max_block=B, max_seqs=len(seq_ctx))
    m.load_weights(torch_tensors(t, "cuda"))
    for i, inp in enumerate(inps):
        m.ingest_seq(i, torch.from_numpy(inp["target_hidden"]))
    ids_b = np.stack([inp["ids"] for inp in inps])
    ids, logits, h = m.draft_batch(ids=torch.from_numpy(ids_b), return_logits=True,
                                   return_hidden=True)
    torch.cuda.synchronize()
    ids, logits, h = ids.cpu().numpy(), logits.cpu().numpy(), h.float().cpu().numpy()
    for i, inp in enumerate(inps):
        h_ref, ids_ref, ids64, ti, tv = _oracle_both(W, inp)
        assert_close_fp16(h[i], h_ref, what=f"split-K batch {seq_ctx} sequence {i} hidden")
        check_argmax(ids[i], logits[i], ids_ref, ids64, f"split-K batch {seq_ctx} sequence {i}",
                     ti, tv, LOGIT_TOL)
    m.close()


def test_batch_full_matches_golden():
    from mirror_sd_amd.dflash import DFlashDraftModel
    name = "llama8b_batch"
    g = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    wl = workload(name)
    cfg = wl.cfg
    print(f"case {name}: generating inputs", flush=True)
    t = synth.make_weights_numpy(cfg, seed=0)
    inps = synth.make_batch_inputs_numpy(cfg, wl.block, wl.seq_ctx, seed=0)
    dig = input_digests(t, {f"{k}.s{i}": v for i, inp in enumerate(inps) for k, v in inp.items()})
    assert dig == dict(zip(g["digest_names"].tolist(), g["digest_values"].tolist()))
    m = DFlashDraftModel(cfg, max_ctx=max(wl.seq_ctx), max_seqs=len(wl.seq_ctx))
    m.load_weights(torch_tensors(t, "cuda"))
    del t
    torch.cuda.empty_cache()
    print(f"case {name}: ingesting {len(inps)} contexts", flush=True)
    for i, inp in enumerate(inps):
        m.ingest_seq(i, torch.from_numpy(inp["target_hidden"]))
    print(f"case {name}: drafting", flush=True)
    ids_b = np.stack([inp["ids"] for inp in inps])
    ids, logits, h = m.draft_batch(ids=torch.from_numpy(ids_b), return_logits=True,
                                   return_hidden=True)
    torch.cuda.synchronize()
    M = ids_b.size
    assert_close_fp16(h.float().cpu().numpy().reshape(M, -1), g["hidden"], what=f"{name} hidden")
    check_argmax(ids.cpu().numpy().reshape(M), logits.cpu().numpy().reshape(M, -1), g["ids"],
                 oracle_alt_runs(g), name, g["top2_idx"], g["top2_val"], LOGIT_TOL)
    m.close()
