"""GPU tests of the parallel caller's pieces (generate.py:1391-1513): the block noise
embedding with the soft anchor (generate.py:1419-1437) through dfl_embed_block, and the
split API (prepare_forward / run_kernels / read_*) running on the draft's own HIP stream
from a worker thread while the caller's stream is busy.

Tolerance of the soft anchor: it is an fp32 softmax-weighted sum of fp16 rows cast to fp16,
so it may differ from the oracle by one fp16 rounding step of the result (exp and the
summation order are not fixed by the reference); the row gather is bit-exact.
"""

import threading

import numpy as np
import pytest

from oracle import dflash_oracle as O
from mirror_sd_amd.config import DFlashConfig, workload
from mirror_sd_amd import synth
from parity_util import torch_tensors

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _embed_model(V, H=256, seed=0):
    from mirror_sd_amd.dflash import DFlashDraftModel
    cfg = DFlashConfig(hidden_size=H, num_hidden_layers=1, intermediate_size=512,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                       vocab_size=V, block_size=16)
    m = DFlashDraftModel(cfg, max_ctx=64)
    E = np.random.default_rng(seed).normal(0, 0.02, (V, H)).astype(np.float16)
    m.load_head(torch.ones(H, dtype=torch.float16), embed=torch.from_numpy(E))
    return m, E


def _fp16_steps(a, b):
    """Distance in fp16 rounding steps at the larger magnitude (1 = neighbouring values)."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    ulp = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float64)
    return np.abs(a - b) / np.maximum(ulp, np.float64(2.0 ** -24))


@pytest.fixture(scope="module")
def vocab_model():
    return _embed_model(151936, H=256)


def test_embed_block_rows_bitexact(vocab_model):
    m, E = vocab_model
    ids = np.array([5, 151935, 0, 77777] + [151669] * 12, dtype=np.int32)
    out = m.embed_block(torch.from_numpy(ids))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out[0].cpu().numpy().view(np.uint16), E[ids].view(np.uint16))


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_soft_anchor_matches_oracle(vocab_model, dtype):
    m, E = vocab_model
    rng = np.random.default_rng({"float32": 1, "float16": 2, "bfloat16": 3}[dtype])
    V = E.shape[0]
    for trial in range(3):
        lg = torch.from_numpy(rng.normal(0, 3, V).astype(np.float32)).to(getattr(torch, dtype))
        ids = np.array([int(rng.integers(V))] + [151669] * 15, dtype=np.int32)
        got = m.embed_block(torch.from_numpy(ids), correction_logits=lg.cuda())[0]
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        want = O.embed_block(E, ids, lg.float().numpy())
        np.testing.assert_array_equal(got[1:].view(np.uint16), want[1:].view(np.uint16))
        steps = _fp16_steps(got[0], want[0])
        assert steps.max() <= 1.0, f"{dtype} trial {trial}: {steps.max()} fp16 steps"


def test_soft_anchor_ties_nan_and_top_k(vocab_model):
    m, E = vocab_model
    V = E.shape[0]
    ids = torch.tensor([3, 4], dtype=torch.int32)
    # every logit equal, a few NaN among the lowest ids: the lowest non-NaN ids win
    lg = np.zeros(V, dtype=np.float32)
    lg[[0, 2]] = np.nan
    for k in (1, 3, 8):
        got = m.embed_block(ids, torch.from_numpy(lg).cuda(), top_k=k)[0, 0].cpu().numpy()
        want = O.soft_anchor(E, lg, top_k=k)
        assert _fp16_steps(got, want).max() <= 1.0, k
    # the top-k spread over the vocabulary (one per scan workgroup slice and the last row)
    lg = np.full(V, -10.0, dtype=np.float32)
    top = [0, 2374, 50000, 50001, 99999, 120000, 151934, 151935]
    lg[top] = np.linspace(1.0, 2.0, 8, dtype=np.float32)
    got = m.embed_block(ids, torch.from_numpy(lg).cuda())[0, 0].cpu().numpy()
    assert _fp16_steps(got, O.soft_anchor(E, lg)).max() <= 1.0
    # a dominant logit selects its row exactly
    lg[99999] = 500.0
    got = m.embed_block(ids, torch.from_numpy(lg).cuda())[0, 0].cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), E[99999].view(np.uint16))


def test_embed_block_rejects_bad_arguments(vocab_model):
    m, E = vocab_model
    V = E.shape[0]
    ids = torch.tensor([1, 2], dtype=torch.int32)
    lg = torch.zeros(V, device="cuda")
    with pytest.raises(ValueError):
        m.embed_block(torch.tensor([V], dtype=torch.int32))
    with pytest.raises(ValueError):
        m.embed_block(ids, lg, top_k=9)
    with pytest.raises(ValueError):
        m.embed_block(ids, lg, top_k=0)
    with pytest.raises(ValueError):
        m.embed_block(ids, torch.zeros(V + 1, device="cuda"))


# ---------------------------------------------------------------------------
# Split API on the draft stream, overlapped with work on the caller's stream
# ---------------------------------------------------------------------------

def test_split_api_on_worker_thread_matches_serial():
    """prepare_forward (main thread) -> run_kernels (worker thread, draft stream) while the
    main stream runs a long matmul chain -> join -> read_output / read_draft_tokens, as
    _spec_generate_parallel does (generate.py:1320-1333, 1391-1513).  Results equal the
    serial __call__ / draft on the same inputs bit for bit (same kernels, same order)."""
    wl, cfg = workload("tiny"), workload("tiny").cfg
    t = synth.make_weights_numpy(cfg, seed=4)
    inp = synth.make_inputs_numpy(cfg, wl.block, wl.ctx, seed=4)
    from mirror_sd_amd.dflash import DFlashDraftModel
    m = DFlashDraftModel(cfg, max_ctx=wl.ctx + 64)
    m.load_weights(torch_tensors(t, "cuda"))
    th = torch.from_numpy(inp["target_hidden"]).cuda()[None]
    ne = m.embed_block(torch.from_numpy(inp["ids"]))
    ref_h = m(ne, th)                                   # serial path, cache=None
    ref_ids = m.draft(torch.from_numpy(inp["ids"]), th)
    torch.cuda.synchronize()
    ref_h, ref_ids = ref_h.cpu(), ref_ids.cpu()
    a = torch.randn(2048, 2048, device="cuda")
    for step in range(3):
        cache = m.make_cache(0, 0)
        m.prepare_forward(ne, m._compute_context(th), cache, th)
        box = {}
        worker = threading.Thread(target=lambda: box.setdefault("r", m.run_kernels()))
        worker.start()
        x = a
        for _ in range(20):                             # "verify" on the caller's stream
            x = torch.tanh(x @ a) * 0.5
        worker.join()
        h = m.read_output()
        ids = m.read_draft_tokens()
        torch.cuda.synchronize()
        assert torch.isfinite(x).all()
        np.testing.assert_array_equal(h.cpu().numpy().view(np.uint16),
                                      ref_h.numpy().view(np.uint16), err_msg=f"step {step}")
        np.testing.assert_array_equal(ids.cpu().numpy().ravel(), ref_ids.numpy())


def test_split_api_rope_offset_from_cache():
    """The ANE-path protocol sets cache.offset = start_pos - ctx_len before prepare_forward
    (generate.py:1409-1417); run_kernels re-ingests the step's target_hidden from there,
    which equals an oracle forward whose cache starts at that offset."""
    wl, cfg = workload("tiny"), workload("tiny").cfg
    t = synth.make_weights_numpy(cfg, seed=5)
    inp = synth.make_inputs_numpy(cfg, wl.block, wl.ctx, seed=5)
    W = O.OracleWeights(cfg, t)
    from mirror_sd_amd.dflash import DFlashDraftModel
    m = DFlashDraftModel(cfg, max_ctx=wl.ctx + 64)
    m.load_weights(torch_tensors(t, "cuda"))
    noise = O.embed(W, inp["ids"]).astype(np.float16)
    off = 37
    oc = [O.OracleKVCache() for _ in range(cfg.num_hidden_layers)]
    for c in oc:
        c.offset = off
    ref = O.draft_forward(W, noise, inp["target_hidden"], cache=oc, fp16=True)
    cache = m.make_cache(0, 0)
    for c in cache:
        c.offset = off
    th = torch.from_numpy(inp["target_hidden"])[None]
    m.prepare_forward(torch.from_numpy(noise)[None], None, cache, th)
    m.run_kernels(wait=False)
    h = m.read_output()
    torch.cuda.synchronize()
    from parity_util import assert_close_fp16
    assert_close_fp16(h[0].float().cpu().numpy(), ref, what="offset 37")
