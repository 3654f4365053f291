"""GPU tests of the drop-in surface of ``DFlashDraftModel`` beyond the fused path:

* scaled RoPE (rope_scaling llama3 / linear, initialize_rope at dflash.py:254-261) against
  the oracle's scaled frequencies, at positions where the scaling changes the result;
* assignable cache tensors and ``update_and_fetch`` (dflash.py:161-177; the cache
  transplant of generate.py:917-941) against the oracle's cache;
* the batch axis of ``__call__`` (B_ > 1, dflash.py:384-403) against one call per sequence;
* device token ids outside the vocabulary: no host read-back, device error bit 0 instead.

Tolerances as everywhere: cosine >= 0.9995, max-abs <= 2e-2 on fp16 hidden states.
"""

import numpy as np
import pytest

from oracle import dflash_oracle as O
from mirror_sd_amd.config import DFlashConfig
from mirror_sd_amd import synth
from parity_util import assert_close_fp16, cos_sim, device_errors, torch_tensors

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _cfg(rope_scaling=None, layers=2, theta=5e5, vocab=1024):
    return DFlashConfig(hidden_size=256, num_hidden_layers=layers, intermediate_size=512,
                        num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                        rope_theta=theta, vocab_size=vocab, block_size=8,
                        mask_token_id=vocab - 1, rope_scaling=rope_scaling)


def _model(cfg, max_ctx=512, **kw):
    from mirror_sd_amd.dflash import DFlashDraftModel
    return DFlashDraftModel(cfg, max_ctx=max_ctx, **kw)


@pytest.mark.parametrize("rs", [
    {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
     "original_max_position_embeddings": 8192},
    {"type": "linear", "factor": 4.0},
])
def test_scaled_rope_matches_oracle(rs):
    """Two steps through a cache whose positions start at 200000 (where llama3's stretched
    low frequencies and linear scaling change every angle): the GPU matches the oracle
    with the same scaling and is far from the unscaled oracle."""
    cfg = _cfg(rs)
    t = synth.make_weights_numpy(cfg, seed=21)
    W = O.OracleWeights(cfg, t)
    cfg0 = _cfg(None)
    W0 = O.OracleWeights(cfg0, t)
    m = _model(cfg)
    m.load_weights(torch_tensors(t, "cuda"))
    cache = m.make_cache(0, 0)
    oc = [O.OracleKVCache() for _ in range(cfg.num_hidden_layers)]
    oc0 = [O.OracleKVCache() for _ in range(cfg.num_hidden_layers)]
    for c in cache + oc + oc0:
        c.offset = 200000
    B = 8
    for step, C in enumerate((96, 40)):
        inp = synth.make_inputs_numpy(cfg, B, C, seed=30 + step)
        noise = O.embed(W, inp["ids"]).astype(np.float16)
        ref = O.draft_forward(W, noise, inp["target_hidden"], cache=oc, fp16=True)
        ref0 = O.draft_forward(W0, noise, inp["target_hidden"], cache=oc0, fp16=True)
        out = m(torch.from_numpy(noise)[None], torch.from_numpy(inp["target_hidden"])[None],
                cache=cache)
        torch.cuda.synchronize()
        got = out[0].float().cpu().numpy()
        assert_close_fp16(got, ref, what=f"{rs} step {step}")
        # the rotated keys show the scaling directly (the hidden states only through the
        # attention): the cache rows match the scaled oracle's, not the unscaled one's
        for layer in range(cfg.num_hidden_layers):
            k = cache[layer].keys[0].float().cpu().numpy()
            assert_close_fp16(k, oc[layer].keys, what=f"{rs} step {step} layer {layer} keys")
            assert cos_sim(k, oc0[layer].keys) < 0.9, "the scaling changed nothing"
        for c in cache + oc + oc0:
            c.trim(B)
    m.close()


def _two_models(cfg, t, **kw):
    a, b = _model(cfg, **kw), _model(cfg, **kw)
    for m in (a, b):
        m.load_weights(torch_tensors(t, "cuda"))
    return a, b


@pytest.mark.parametrize("sink,window", [(0, 0), (16, 96)])
def test_cache_transplant_matches_continuing_model(sink, window):
    """generate.py:917-941 moves a draft cache between models by assigning keys, values
    and offset.  Model A runs two steps; its cache is transplanted into model B's fresh
    cache; both then draft a third step: identical hidden states, and both match the
    oracle's cache run.  With a sink + window, the assigned rows are already windowed."""
    cfg = _cfg(None)
    t = synth.make_weights_numpy(cfg, seed=22)
    W = O.OracleWeights(cfg, t)
    A, Bm = _two_models(cfg, t)
    ca = A.make_cache(sink, window)
    oc = [O.OracleKVCache(sink, window) for _ in range(cfg.num_hidden_layers)]
    B = 8
    steps = [synth.make_inputs_numpy(cfg, B, C, seed=40 + i) for i, C in enumerate((70, 50, 30))]

    def run(model, cache, inp):
        noise = O.embed(W, inp["ids"]).astype(np.float16)
        out = model(torch.from_numpy(noise)[None], torch.from_numpy(inp["target_hidden"])[None],
                    cache=cache)
        torch.cuda.synchronize()
        return out[0].float().cpu().numpy()

    for inp in steps[:2]:
        run(A, ca, inp)
        for c in ca:
            c.trim(B)
        O.draft_forward(W, O.embed(W, inp["ids"]).astype(np.float16), inp["target_hidden"],
                        cache=oc, fp16=True)
        for c in oc:
            c.trim(B)
    cb = Bm.make_cache(sink, window)
    for c_old, c_new in zip(ca, cb):     # the transplant, as generate.py:922-926
        c_new.keys = c_old.keys
        c_new.values = c_old.values
        c_new.offset = c_old.offset
    assert all(c.keys.shape == (1, 2, oc[0].keys.shape[1], 128) for c in cb)
    ha = run(A, ca, steps[2])
    hb = run(Bm, cb, steps[2])
    if window == 0:   # the same rows in the same cache order: the same bits
        np.testing.assert_array_equal(ha, hb)
    else:             # A's window is a wrapped ring, B's in order: the same keys, summed
        assert_close_fp16(hb, ha, what="transplanted vs continuing")   # in another order
    ref = O.draft_forward(W, O.embed(W, steps[2]["ids"]).astype(np.float16),
                          steps[2]["target_hidden"], cache=oc, fp16=True)
    assert_close_fp16(hb, ref, what=f"transplanted sink={sink} window={window}")
    # and back (c_old.keys = c_new.keys): A's cache holds B's rows
    for c in cb:
        c.trim(B)
    for c_old, c_new in zip(ca, cb):
        c_old.keys = c_new.keys
        c_old.values = c_new.values
        c_old.offset = c_new.offset
    for c_old, c_new in zip(ca, cb):
        np.testing.assert_array_equal(c_old.keys.cpu().numpy(), c_new.keys.cpu().numpy())
    A.close()
    Bm.close()


def test_update_and_fetch_matches_oracle_cache():
    """update_and_fetch (dflash.py:168-177) on the handles: rows appended to the device
    cache's rows, offset advanced, the window applied; the next forward attends to them.
    The oracle's cache gets the same rows."""
    cfg = _cfg(None)
    t = synth.make_weights_numpy(cfg, seed=23)
    W = O.OracleWeights(cfg, t)
    m = _model(cfg)
    m.load_weights(torch_tensors(t, "cuda"))
    sink, window = 8, 48
    cache = m.make_cache(sink, window)
    oc = [O.OracleKVCache(sink, window) for _ in range(cfg.num_hidden_layers)]
    B = 8
    inp = synth.make_inputs_numpy(cfg, B, 40, seed=50)
    noise = O.embed(W, inp["ids"]).astype(np.float16)
    m(torch.from_numpy(noise)[None], torch.from_numpy(inp["target_hidden"])[None], cache=cache)
    torch.cuda.synchronize()
    O.draft_forward(W, noise, inp["target_hidden"], cache=oc, fp16=True)
    for c in cache + oc:
        c.trim(B)
    rng = np.random.default_rng(7)
    extra = [(rng.standard_normal((2, 20, 128)).astype(np.float16),
              rng.standard_normal((2, 20, 128)).astype(np.float16)) for _ in cache]
    for c, o, (k, v) in zip(cache, oc, extra):
        kk, vv = c.update_and_fetch(torch.from_numpy(k)[None].cuda(), torch.from_numpy(v)[None].cuda())
        ok, ov = o.update_and_fetch(k.astype(np.float64), v.astype(np.float64))
        assert kk.shape[2] == ok.shape[1] == sink + window and c.offset == o.offset
        # the appended rows exactly, the rows the forward computed within the tolerance
        np.testing.assert_array_equal(kk[0, :, -20:].float().cpu().numpy(), ok[:, -20:])
        np.testing.assert_array_equal(vv[0, :, -20:].float().cpu().numpy(), ov[:, -20:])
        assert_close_fp16(kk[0, :, :-20].float().cpu().numpy(), ok[:, :-20], what="kept keys")
        assert_close_fp16(vv[0, :, :-20].float().cpu().numpy(), ov[:, :-20], what="kept values")
    inp2 = synth.make_inputs_numpy(cfg, B, 16, seed=51)
    noise2 = O.embed(W, inp2["ids"]).astype(np.float16)
    out = m(torch.from_numpy(noise2)[None], torch.from_numpy(inp2["target_hidden"])[None],
            cache=cache)
    torch.cuda.synchronize()
    ref = O.draft_forward(W, noise2, inp2["target_hidden"], cache=oc, fp16=True)
    assert_close_fp16(out[0].float().cpu().numpy(), ref, what="after update_and_fetch")
    for c, o in zip(cache, oc):
        np.testing.assert_array_equal(c.keys.shape[2], o.keys.shape[1])
    m.close()


def test_batch_axis_matches_single_sequence_calls():
    """__call__ with [B_, q, H] / [B_, C, nf*H] (B_ = 3, ragged contexts not allowed by the
    reference's tensors, so equal C) through a cache over two steps: each sequence matches
    the oracle run on it alone; the cache handles show [B_, NKV, L, D]."""
    cfg = _cfg(None)
    t = synth.make_weights_numpy(cfg, seed=24)
    W = O.OracleWeights(cfg, t)
    n = 3
    m = _model(cfg, max_seqs=n)
    m.load_weights(torch_tensors(t, "cuda"))
    cache = m.make_cache(0, 0)
    oc = [[O.OracleKVCache() for _ in range(cfg.num_hidden_layers)] for _ in range(n)]
    B = 8
    for step, C in enumerate((64, 24)):
        ins = [synth.make_inputs_numpy(cfg, B, C, seed=60 + 10 * step + s) for s in range(n)]
        noise = np.stack([O.embed(W, i["ids"]).astype(np.float16) for i in ins])
        th = np.stack([i["target_hidden"] for i in ins])
        out = m(torch.from_numpy(noise), torch.from_numpy(th), cache=cache)
        torch.cuda.synchronize()
        assert tuple(out.shape) == (n, B, cfg.hidden_size)
        for s in range(n):
            ref = O.draft_forward(W, noise[s], th[s], cache=oc[s], fp16=True)
            assert_close_fp16(out[s].float().cpu().numpy(), ref, what=f"step {step} seq {s}")
            for c in oc[s]:
                c.trim(B)
        assert tuple(cache[0].keys.shape) == (n, 2, C + B + (64 if step else 0), 128)
        for c in cache:
            c.trim(B)
    # no cache: independent one-shot forwards
    ins = [synth.make_inputs_numpy(cfg, B, 32, seed=90 + s) for s in range(n)]
    noise = np.stack([O.embed(W, i["ids"]).astype(np.float16) for i in ins])
    th = np.stack([i["target_hidden"] for i in ins])
    out = m(torch.from_numpy(noise), torch.from_numpy(th))
    torch.cuda.synchronize()
    for s in range(n):
        assert_close_fp16(out[s].float().cpu().numpy(),
                          O.draft_forward(W, noise[s], th[s], fp16=True), what=f"no cache seq {s}")
    with pytest.raises(ValueError):
        m(torch.from_numpy(np.concatenate([noise, noise[:1]])),
          torch.from_numpy(np.concatenate([th, th[:1]])))   # 4 sequences > max_seqs
    m.close()


def test_device_ids_out_of_range_flag_without_host_sync():
    """Token ids already on the device are not read back by the host: an id outside the
    vocabulary raises nothing at the call, sets device error bit 0 and drafts from a zero
    row; host ids outside the vocabulary raise ValueError."""
    cfg = _cfg(None, layers=1)
    t = synth.make_weights_numpy(cfg, seed=25)
    m = _model(cfg)
    m.load_weights(torch_tensors(t, "cuda"))
    inp = synth.make_inputs_numpy(cfg, 8, 16, seed=70)
    ids = torch.from_numpy(inp["ids"]).cuda()
    m.draft(ids, torch.from_numpy(inp["target_hidden"]))
    torch.cuda.synchronize()
    assert device_errors(m) == 0
    bad = ids.clone()
    bad[3] = cfg.vocab_size + 5
    m.draft(bad, torch.from_numpy(inp["target_hidden"]))
    torch.cuda.synchronize()
    assert device_errors(m) & 1
    with pytest.raises(ValueError):
        m.draft(bad.cpu(), torch.from_numpy(inp["target_hidden"]))
    m.close()


def _chi2_pvalue(counts, probs):
    """Pearson chi-square goodness of fit of counts against probs, categories with an
    expected count below 5 lumped together; returns the p-value."""
    from scipy.stats import chi2
    n = counts.sum()
    exp = probs * n
    big = exp >= 5
    obs = np.append(counts[big], counts[~big].sum())
    e = np.append(exp[big], exp[~big].sum())
    keep = e > 0
    stat = float(((obs[keep] - e[keep]) ** 2 / e[keep]).sum())
    return float(chi2.sf(stat, keep.sum() - 1))


@pytest.mark.parametrize("V,n_seq,B", [(1024, 1, 8), (32768, 1, 8), (1024, 3, 32)])
def test_sampling_matches_softmax(V, n_seq, B):
    """set_sampling(T): the draft ids are draws from softmax(logits / T) per row -- the
    categorical of sample() (dflash.py:133-136).  Over 600 seeds, each row's counts fit
    softmax(logits / T) of the same call's returned logits (chi-square, Bonferroni over
    rows); a fixed seed repeats its draws; T below 1e-5 gives the argmax.  Shapes: the plain
    stream-K lm_head (V 1024), the balanced one (V 32768), the stacked tile GEMM (3 x 32
    rows)."""
    cfg = _cfg(None, layers=1, vocab=V)
    cfg.block_size = B
    t = synth.make_weights_numpy(cfg, seed=26)
    m = _model(cfg, max_ctx=64, max_seqs=n_seq)
    m.load_weights(torch_tensors(t, "cuda"))
    rng = np.random.default_rng(27)
    ids = torch.from_numpy(rng.integers(0, V, (n_seq, B)).astype(np.int32)).cuda()
    for s in range(n_seq):
        m.ingest_seq(s, torch.from_numpy(synth.np_normal(28 + s, "th", (16, 5 * 256), 1.0,
                                                         np.float16)))

    def call(T, seed, logits=False):
        r = m.draft_batch(ids=ids, return_logits=logits, temperature=T, seed=seed)
        return r

    g, lg = call(0.0, 0, logits=True)
    lg = lg.reshape(n_seq * B, V).double().cpu().numpy()
    np.testing.assert_array_equal(g.reshape(-1).cpu().numpy(), np.argmax(lg, axis=1))
    np.testing.assert_array_equal(call(1e-6, 5).cpu().numpy(), g.cpu().numpy())
    T = float(np.median(lg.std(axis=1))) / 3.0   # logits / T spread ~ 3: a few dozen likely ids
    a1, a2 = call(T, 123).cpu().numpy(), call(T, 123).cpu().numpy()
    np.testing.assert_array_equal(a1, a2)
    N = 600
    draws = np.stack([call(T, 1000 + i).reshape(-1).cpu().numpy() for i in range(N)])
    rows = n_seq * B
    p_min = 1.0
    for r in range(rows):
        p = np.exp((lg[r] - lg[r].max()) / T)
        p /= p.sum()
        counts = np.bincount(draws[:, r], minlength=V).astype(np.float64)
        p_min = min(p_min, _chi2_pvalue(counts, p))
    assert p_min * rows > 1e-3, f"a row's draws do not fit softmax(logits / T): p = {p_min}"
    assert len(np.unique(draws[:, 0])) > 3   # the samples are not the argmax
    m.close()
