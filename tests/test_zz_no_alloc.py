"""The allocation-free block embedding (dfl_embed_block_noalloc) against the context entry
point dfl_embed_block: the same kernels, so the same bits, on two calls in a row (the second
with fewer rows, a shorter logits vector and a smaller top_k), then an out-of-range id that
must set error bit 0 in the caller's word and give a zero row."""

import ctypes

import numpy as np
import pytest

from mirror_sd_amd import _lib
from mirror_sd_amd.config import DFlashConfig

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _model(V, H, seed=0):
    from mirror_sd_amd.dflash import DFlashDraftModel
    cfg = DFlashConfig(hidden_size=H, num_hidden_layers=1, intermediate_size=512,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                       vocab_size=V, block_size=16)
    m = DFlashDraftModel(cfg, max_ctx=64)
    E = np.random.default_rng(seed).normal(0, 0.02, (V, H)).astype(np.float16)
    m.load_head(torch.ones(H, dtype=torch.float16), embed=torch.from_numpy(E))
    return m, torch.from_numpy(E).cuda()


def _noalloc(E, ids, logits, top_k, err):
    L = _lib.load()
    V_emb, H = E.shape
    out = torch.full((ids.numel(), H), float("nan"), dtype=torch.float16, device="cuda")
    code, V = 0, 0
    if logits is not None:
        code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[logits.dtype]
        V = logits.numel()
    _lib.check(L.dfl_embed_block_noalloc(ids.data_ptr(), ids.numel(), E.data_ptr(), V_emb, H,
                                         _lib.ptr(logits), code, V, top_k, out.data_ptr(),
                                         err.data_ptr(), _lib.stream_handle()),
               "dfl_embed_block_noalloc")
    return out


def test_noalloc_embed_block_matches_context_entry_point():
    V, H = 151936, 512
    m, E = _model(V, H)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cpu").manual_seed(7)
    cases = [  # (rows, logits length, logits dtype, top_k)
        (32, V, torch.float32, 8),
        (5, 40000, torch.float16, 3),
    ]
    for B, Vl, dt, k in cases:
        print(f"noalloc case B={B} V={Vl} {dt} top_k={k}", flush=True)
        ids = torch.randint(0, V, (B,), generator=g, dtype=torch.int32).cuda()
        lg = (torch.randn(Vl, generator=g) * 3).to(dt).cuda()
        want = m.embed_block(ids, correction_logits=lg, top_k=k)[0]
        got = _noalloc(E, ids, lg, k, err)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16),
                                      want.cpu().numpy().view(np.uint16))
        # rows past the anchor are plain gathers of the embedding
        np.testing.assert_array_equal(got[1:].cpu().numpy().view(np.uint16),
                                      E[ids[1:].long()].cpu().numpy().view(np.uint16))
    # without logits: every row is a gather
    ids = torch.tensor([3, V - 1, 0], dtype=torch.int32).cuda()
    got = _noalloc(E, ids, None, 8, err)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16),
                                  E[ids.long()].cpu().numpy().view(np.uint16))
    assert int(err.item()) == 0
    # an id outside [0, Vemb) gives a zero row and error bit 0 in the caller's word
    ids = torch.tensor([1, V], dtype=torch.int32).cuda()
    got = _noalloc(E, ids, None, 8, err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    assert not got[1].float().abs().sum().item()
    m.close()


def test_noalloc_embed_block_rejects_bad_arguments():
    L = _lib.load()
    E = torch.zeros((64, 256), dtype=torch.float16, device="cuda")
    ids = torch.zeros(4, dtype=torch.int32, device="cuda")
    out = torch.empty((4, 256), dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    lg = torch.zeros(64, dtype=torch.float32, device="cuda")
    s = _lib.stream_handle()
    assert L.dfl_embed_block_noalloc(ids.data_ptr(), 4, E.data_ptr(), 64, 256, lg.data_ptr(), 0,
                                     64, 9, out.data_ptr(), err.data_ptr(), s) == _lib.DFL_EINVAL
    assert b"top_k" in L.dfl_last_error()
    assert L.dfl_embed_block_noalloc(ids.data_ptr(), 4, E.data_ptr(), 64, 256, lg.data_ptr(), 0,
                                     65, 8, out.data_ptr(), err.data_ptr(), s) == _lib.DFL_EINVAL
    assert L.dfl_embed_block_noalloc(ids.data_ptr(), 4, E.data_ptr(), 64, 256, None, 0, 0, 8,
                                     out.data_ptr(), None, s) == _lib.DFL_EINVAL
