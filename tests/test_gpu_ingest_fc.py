"""Prompt-sized context ingest (more than 64 rows, dflash.py:122-130 + 287-294): the rows
of the concatenated target_hidden, of the tapped layers or of strided slices of wider
buffers (any alignment) are gathered into fragment layout and the fc fusion projection
runs on the tile GEMM over the packed fp16 fc weight.  Every variant matches the oracle
within the draft tolerance, its argmax ids pass the suite's agreement rule (check_argmax:
a row may differ only where the oracle's fp32 and fp64 runs disagree), and the variants
agree with each other within
SAME_TOL.  The per-step ingest's fc (at most 64 rows, the stream-K kernel) reads up to 16
aligned rows in place and gathers the rest first: both give the same bits."""

import numpy as np
import pytest

from oracle import dflash_oracle as O
from mirror_sd_amd import synth
from mirror_sd_amd.config import _draft_cfg
from parity_util import assert_close_fp16, check_argmax, torch_tensors

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SAME_TOL = dict(cos_min=0.99999, max_abs=4e-3)
LOGIT_TOL = 2e-2
CTX = 200   # a partial last m-tile


@pytest.fixture(scope="module")
def case():
    from mirror_sd_amd.dflash import DFlashDraftModel
    cfg = _draft_cfg(256, 4, 2, 512, 2, vocab=1024, block=8)
    t = synth.make_weights_numpy(cfg, seed=11)
    inp = synth.make_inputs_numpy(cfg, 8, CTX, seed=11)
    m = DFlashDraftModel(cfg, max_ctx=CTX + 64)
    m.load_weights(torch_tensors(t, "cuda"))
    W = O.OracleWeights(cfg, t)
    # the oracle's fp32-accumulation run (ids, top-2 logits) and its fp64 run's ids
    h_ref, lg, ids_ref = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True,
                                       dtype=np.float32)
    _, _, ids64 = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True)
    ti = np.argsort(-lg, axis=-1, kind="stable")[:, :2]
    th = torch.from_numpy(inp["target_hidden"]).cuda()
    return dict(cfg=cfg, m=m, inp=inp, th=th, h_ref=h_ref, ids_ref=ids_ref, ids64=ids64,
                ti=ti, tv=np.take_along_axis(lg, ti, -1))


def _misaligned(x):
    """The same values at a data pointer 2 bytes past a 16-byte boundary."""
    buf = torch.zeros(x.numel() + 8, dtype=torch.float16, device=x.device)
    v = buf[1:1 + x.numel()].view(x.shape)
    v.copy_(x)
    assert v.data_ptr() % 16 == 2
    return v


def _check(case, src, what, h_base=None):
    m, inp = case["m"], case["inp"]
    ids = torch.from_numpy(inp["ids"])
    i, lg, h = m.draft(ids, src, return_logits=True, return_hidden=True)
    torch.cuda.synchronize()
    assert_close_fp16(h.float().cpu().numpy(), case["h_ref"], what=what)
    check_argmax(i.cpu().numpy(), lg.cpu().numpy(), case["ids_ref"], case["ids64"],
                 f"prompt fc: {what}", case["ti"], case["tv"], LOGIT_TOL)
    if h_base is not None:
        assert_close_fp16(h.float().cpu().numpy(), h_base, what=what + " vs concatenated",
                          **SAME_TOL)
    return h.float().cpu().numpy()


def test_prompt_fc_concatenated_features_and_strided(case):
    cfg, th = case["cfg"], case["th"]
    H = cfg.hidden_size
    nf = th.shape[1] // H
    h0 = _check(case, th, "concatenated target_hidden")
    feats = [th[:, j * H:(j + 1) * H].contiguous()[None] for j in range(nf)]
    _check(case, feats, "tapped-layer list", h0)
    wide = [torch.zeros((1, CTX, 3 * H), dtype=torch.float16, device="cuda") for _ in feats]
    for w, f in zip(wide, feats):
        w[:, :, H:2 * H] = f
    _check(case, [w[:, :, H:2 * H] for w in wide], "strided tapped layers", h0)


def test_prompt_fc_unaligned_rows(case):
    cfg, th = case["cfg"], case["th"]
    H = cfg.hidden_size
    nf = th.shape[1] // H
    h0 = _check(case, th, "concatenated target_hidden")
    _check(case, _misaligned(th), "unaligned target_hidden", h0)
    # the feature-list ABI takes aligned rows only: the wrapper copies unaligned ones
    feats = [_misaligned(th[:, j * H:(j + 1) * H].contiguous())[None] for j in range(nf)]
    _check(case, feats, "unaligned tapped layers (copied by the wrapper)", h0)


@pytest.mark.parametrize("k", [1, 5, 16, 17, 32])
def test_step_fc_rows_read_in_place_match_gathered(k):
    """Per-step ingest (at most 64 rows: the stream-K fc).  Up to 16 rows whose data is
    16-byte aligned are read in place, row-major, by the fc; unaligned rows (and more than
    16) are gathered into fragment layout first.  The same values reach the same products,
    so the K/V caches of every layer and the next block's hidden states agree bit for bit;
    the tapped-layer list (strided, aligned) takes the in-place path too."""
    from mirror_sd_amd.dflash import DFlashDraftModel
    cfg = _draft_cfg(256, 4, 2, 512, 2, vocab=1024, block=8)
    H, nf, C0 = cfg.hidden_size, 5, 40
    t = synth.make_weights_numpy(cfg, seed=13)
    th0 = torch.from_numpy(synth.np_normal(13, "step.ctx", (C0, nf * H), 1.0, np.float16)).cuda()
    th1 = torch.from_numpy(synth.np_normal(13, f"step.rows{k}", (k, nf * H), 1.0, np.float16)).cuda()
    wide = torch.zeros((nf, k, 3 * H), dtype=torch.float16, device="cuda")
    for j in range(nf):
        wide[j, :, H:2 * H] = th1[:, j * H:(j + 1) * H]
    srcs = {"aligned": th1[None], "unaligned": _misaligned(th1)[None],
            "strided tapped layers": [wide[j, :, H:2 * H][None] for j in range(nf)]}
    ids = np.array([7] + [cfg.mask_token_id] * (cfg.block_size - 1), dtype=np.int32)
    res = {}
    for name, src in srcs.items():
        print(f"step ingest of {k} rows: {name}", flush=True)
        m = DFlashDraftModel(cfg, max_ctx=C0 + 64)
        m.load_weights(torch_tensors(t, "cuda"))
        cache = m.make_cache(0, 0)
        noise = m.embed_block(torch.from_numpy(ids).cuda())
        noise = noise if noise.dim() == 3 else noise[None]
        m(noise, th0[None], cache=cache)
        for c in cache:
            c.trim(cfg.block_size)
        out = m(noise, src, cache=cache)
        torch.cuda.synchronize()
        kv = [(kk[:, :C0 + k].float().cpu().numpy(), vt[:, :, :C0 + k].float().cpu().numpy())
              for kk, vt in m._cache_tensors]
        res[name] = (kv, out.float().cpu().numpy())
    base_kv, base_out = res["unaligned"]
    for name in ("aligned", "strided tapped layers"):
        kv, out = res[name]
        for l, ((k1, v1), (k2, v2)) in enumerate(zip(kv, base_kv)):
            np.testing.assert_array_equal(k1.view(np.uint32), k2.view(np.uint32), err_msg=f"{name} K layer {l}")
            np.testing.assert_array_equal(v1.view(np.uint32), v2.view(np.uint32), err_msg=f"{name} Vt layer {l}")
        np.testing.assert_array_equal(out.view(np.uint32), base_out.view(np.uint32), err_msg=f"{name} hidden")
