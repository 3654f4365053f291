"""A local safetensors checkpoint through load_dflash_model (loader.py:20-116) into the GPU
model: the draft equals the oracle run on the bf16-rounded weights (the reference loader's
cast) within the draft tolerance, and equals bit for bit the model loaded directly from
those rounded tensors."""

import json

import numpy as np
import pytest

from oracle import dflash_oracle as O
from mirror_sd_amd import synth
from mirror_sd_amd.config import workload
from parity_util import assert_close_fp16, torch_tensors

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def test_checkpoint_dir_loads_and_drafts(tmp_path):
    from safetensors.torch import save_file
    from mirror_sd_amd.dflash import DFlashDraftModel
    from mirror_sd_amd.loader import load_dflash_model
    wl = workload("tiny")
    cfg = wl.cfg
    t = synth.make_weights_numpy(cfg, seed=7)
    inp = synth.make_inputs_numpy(cfg, wl.block, wl.ctx, seed=7)
    head = {k: t.pop(k) for k in ("embed_tokens.weight", "lm_head.weight")}
    # fp32 checkpoint in two shards with an index
    tt = {k: torch.from_numpy(v.astype(np.float32)) for k, v in t.items()}
    names = sorted(tt)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half],
              "model-00002-of-00002.safetensors": names[half:]}
    for fname, ns in shards.items():
        save_file({n: tt[n] for n in ns}, str(tmp_path / fname))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"weight_map": {n: f for f, ns in shards.items() for n in ns}}))
    (tmp_path / "config.json").write_text(json.dumps({
        "hidden_size": cfg.hidden_size, "num_hidden_layers": cfg.num_hidden_layers,
        "intermediate_size": cfg.intermediate_size,
        "num_attention_heads": cfg.num_attention_heads,
        "num_key_value_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim,
        "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
        "vocab_size": cfg.vocab_size,
        "dflash_config": {"block_size": cfg.block_size, "mask_token_id": cfg.mask_token_id,
                          "target_layer_ids": cfg.target_layer_ids}}))
    emb = torch.from_numpy(head["embed_tokens.weight"]).cuda()
    lmh = torch.from_numpy(head["lm_head.weight"]).cuda()
    m, lcfg = load_dflash_model(tmp_path, embed_tokens=emb, lm_head=lmh, max_ctx=wl.ctx)
    assert lcfg.target_layer_ids == cfg.target_layer_ids and lcfg.block_size == cfg.block_size
    ids, h = m.draft(torch.from_numpy(inp["ids"]), torch.from_numpy(inp["target_hidden"]),
                     return_hidden=True)
    torch.cuda.synchronize()
    # the oracle on the weights as the loader rounds them (fp32 -> bf16)
    tb = {k: torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).float().numpy()
          for k, v in t.items()}
    tb = {k: (v if k.split(".")[-2].endswith("proj") else v.astype(np.float16))
          for k, v in tb.items()}
    tb.update(head)
    W = O.OracleWeights(lcfg, tb)
    h_ref, _, ids_ref = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True)
    assert_close_fp16(h.float().cpu().numpy(), h_ref, what="loaded checkpoint")
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    # same tensors loaded directly: identical results
    m2 = DFlashDraftModel(lcfg, max_ctx=wl.ctx)
    m2.load_weights(torch_tensors(tb, "cuda"))
    ids2, h2 = m2.draft(torch.from_numpy(inp["ids"]), torch.from_numpy(inp["target_hidden"]),
                        return_hidden=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(h.cpu().numpy().view(np.uint16), h2.cpu().numpy().view(np.uint16))
    np.testing.assert_array_equal(ids.cpu().numpy(), ids2.cpu().numpy())
