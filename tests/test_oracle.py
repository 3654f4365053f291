"""Pins the CPU oracle (oracle/dflash_oracle.py) without the reference's MLX.

The reference ships no golden vectors or known-answer tests for this path, so
each oracle function is pinned here by closed forms, invariants, brute force
on tiny inputs, or an independent library routine (torch CPU float64), each
chosen so that a plausible slip (dropped term, wrong sign, swapped half,
transposed operand, wrong GQA mapping, wrong RoPE position) fails.
"""

import math

import numpy as np
import pytest
import torch

from oracle import dflash_oracle as O
from mirror_sd_amd.config import DFlashConfig


def small_cfg(H=16, NH=4, NKV=2, D=8, F=24, L=2, V=64, theta=1e6):
    return DFlashConfig(hidden_size=H, num_hidden_layers=L, intermediate_size=F,
                        num_attention_heads=NH, num_key_value_heads=NKV, head_dim=D,
                        rope_theta=theta, vocab_size=V, block_size=4,
                        target_layer_ids=[1, 2])


# ---------------------------------------------------------------------------
# W8A16 quantiser (ane_model.py:265-279)
# ---------------------------------------------------------------------------

def test_quantize_roundtrip_bound():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float32)
    q, s = O.quantize_w8(w)
    assert q.dtype == np.int8 and s.dtype == np.float16 and q.shape == w.shape
    s32 = np.abs(w).max(axis=1) / np.float32(127)
    # |w - q*s32| <= s32/2 with the fp32 scale used for rounding
    err = np.abs(w - q.astype(np.float64) * s32[:, None])
    assert np.all(err <= s32[:, None] / 2 * (1 + 1e-6))
    # each row reaches +-127 exactly at its absmax element
    am = np.abs(w).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(64), am]) == 127)
    assert np.abs(q).max() <= 127


def test_quantize_zero_row_and_half_even():
    w = np.zeros((3, 8), dtype=np.float32)
    # row 1: max 127 -> scale exactly 1.0, so w/scale = w; .5 cases round half-even
    w[1] = [127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -126.5]
    w[2] = [-1.0, 0, 0, 0, 0, 0, 0, 0]
    q, s = O.quantize_w8(w)
    assert np.all(q[0] == 0) and s[0] == np.float16(np.float32(1.0) / np.float32(127))
    assert list(q[1]) == [127, 2, 4, -2, 0, 0, 2, -126]
    assert s[1] == np.float16(1.0)
    assert q[2, 0] == -127


def test_quantize_byte_layout():
    w = np.arange(12, dtype=np.float32).reshape(3, 4) - 5
    q, s = O.quantize_w8(w)
    b = q.tobytes()
    assert len(b) == 12 and np.frombuffer(b, dtype=np.int8).reshape(3, 4).tolist() == q.tolist()
    sb = s.tobytes()
    assert np.frombuffer(sb, dtype="<f2").tolist() == s.tolist()


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def test_rmsnorm_closed_forms():
    g = np.linspace(0.5, 2.0, 32)
    for c in (3.0, -0.25):
        y = O.rms_norm(np.full((1, 32), c), g, 1e-6, fp16=False)
        np.testing.assert_allclose(y[0], np.sign(c) * g * abs(c) / math.sqrt(c * c + 1e-6),
                                   rtol=1e-14)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 32))
    # scale invariance (eps -> 0)
    np.testing.assert_allclose(O.rms_norm(7.0 * x, g, 0.0, False), O.rms_norm(x, g, 0.0, False),
                               rtol=1e-12)
    # library cross-check
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (32,), torch.from_numpy(g), eps=1e-6)
    np.testing.assert_allclose(O.rms_norm(x, g, 1e-6, False), ref.numpy(), rtol=1e-12)
    # output has unit rms when g = 1
    y = O.rms_norm(x, np.ones(32), 0.0, False)
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1.0, rtol=1e-12)


def test_head_norm_heads_independent():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 4, 8))
    g = rng.standard_normal(8)
    y = O.head_rms_norm(x, g, 1e-6, False)
    perm = [2, 0, 3, 1]
    np.testing.assert_allclose(O.head_rms_norm(x[:, perm], g, 1e-6, False), y[:, perm])
    for h in range(4):
        np.testing.assert_allclose(y[:, h], O.rms_norm(x[:, h], g, 1e-6, False))


# ---------------------------------------------------------------------------
# neox RoPE
# ---------------------------------------------------------------------------

def test_rope_identity_and_norm_preservation():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 3, 16))
    y0 = O.rope_neox(x, np.zeros(5, dtype=np.int64), 1e4, False)
    np.testing.assert_allclose(y0, x, atol=0)
    y = O.rope_neox(x, np.arange(5) * 977, 1e4, False)
    # each (j, j+8) pair keeps its norm
    n_in = x[..., :8] ** 2 + x[..., 8:] ** 2
    n_out = y[..., :8] ** 2 + y[..., 8:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-12)


def test_rope_complex_form_and_hand_example():
    rng = np.random.default_rng(5)
    D, theta = 16, 1e6
    x = rng.standard_normal((4, 2, D))
    pos = np.array([0, 1, 100, 4097])
    y = O.rope_neox(x, pos, theta, False)
    z = x[..., :D // 2] + 1j * x[..., D // 2:]
    j = np.arange(D // 2)
    rot = np.exp(1j * pos[:, None] * theta ** (-2.0 * j / D))[:, None, :]
    zr = z * rot
    np.testing.assert_allclose(y[..., :D // 2], zr.real, atol=1e-12)
    np.testing.assert_allclose(y[..., D // 2:], zr.imag, atol=1e-12)
    # hand example: D=4, theta=100 -> inv_freq = [1, 0.1]; position 1
    x4 = np.array([[[1.0, 2.0, 3.0, 4.0]]])
    y4 = O.rope_neox(x4, np.array([1]), 100.0, False)[0, 0]
    c0, s0, c1, s1 = math.cos(1), math.sin(1), math.cos(0.1), math.sin(0.1)
    exp = [1 * c0 - 3 * s0, 2 * c1 - 4 * s1, 3 * c0 + 1 * s0, 4 * c1 + 2 * s1]
    np.testing.assert_allclose(y4, exp, rtol=1e-14)


def test_rope_llama3_frequency_bands():
    """Llama 3.1 frequency scaling (mlx_lm Llama3RoPE, the reference's initialize_rope with
    rope_type llama3): frequencies whose wavelength 2 pi / f is below L0 / hf are unchanged,
    above L0 / lf divided by the factor, and the band between interpolated; the interpolation
    meets both neighbours at the band edges (s = 0 -> f / factor, s = 1 -> f), stays
    between them and falls monotonically with j; linear scaling divides every frequency."""
    D, theta, fac, L0, lf, hf = 128, 5e5, 8.0, 8192, 1.0, 4.0
    rs = {"rope_type": "llama3", "factor": fac, "low_freq_factor": lf, "high_freq_factor": hf,
          "original_max_position_embeddings": L0}
    base = O.rope_inv_freq(D, theta)
    got = O.rope_inv_freq(D, theta, rs)
    wl = 2 * np.pi / base
    hi, lo = wl < L0 / hf, wl > L0 / lf
    mid = ~hi & ~lo
    assert hi.sum() > 10 and lo.sum() > 10 and mid.sum() >= 3   # all three bands occur
    np.testing.assert_array_equal(got[hi], base[hi])
    np.testing.assert_allclose(got[lo], base[lo] / fac, rtol=1e-15)
    assert np.all(got[mid] < base[mid]) and np.all(got[mid] > base[mid] / fac)
    assert np.all(np.diff(got) < 0)
    # band edges: a frequency at wavelength exactly L0 / hf (s = 1) keeps its value, at L0 / lf
    # (s = 0) the interpolation gives f / factor
    for w_edge, want in [(L0 / hf, 1.0), (L0 / lf, 1.0 / fac)]:
        f = 2 * np.pi / w_edge
        s = (L0 / w_edge - lf) / (hf - lf)
        assert abs(((1 - s) / fac + s) - want) < 1e-15
    # hand value: the first frequency of the band, computed from the scheme's definition
    j = int(np.argmax(mid))
    s = (L0 * base[j] / (2 * np.pi) - lf) / (hf - lf)
    assert abs(got[j] - base[j] * ((1 - s) / fac + s)) < 1e-18
    np.testing.assert_allclose(O.rope_inv_freq(D, theta, {"type": "linear", "factor": 4.0}),
                               base / 4.0, rtol=1e-15)
    with pytest.raises(NotImplementedError):
        O.rope_inv_freq(D, theta, {"rope_type": "yarn", "factor": 4.0})


def test_rope_relative_position():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 1, 32))
    k = rng.standard_normal((1, 1, 32))
    dots = []
    for p, s in [(10, 3), (1007, 1000), (57, 50)]:
        qr = O.rope_neox(q, np.array([p]), 1e6, False)
        kr = O.rope_neox(k, np.array([s]), 1e6, False)
        dots.append(float((qr * kr).sum()))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-9)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------

def test_sdpa_single_key_and_identical_keys():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((4, 3, 8))
    k1 = rng.standard_normal((2, 1, 8))
    v1 = rng.standard_normal((2, 1, 8))
    o = O.sdpa_gqa(q, k1, v1, 8 ** -0.5, False)
    for h in range(4):
        np.testing.assert_allclose(o[h], np.broadcast_to(v1[h // 2], (3, 8)), rtol=1e-14)
    kk = np.repeat(rng.standard_normal((2, 1, 8)), 5, axis=1)
    vv = rng.standard_normal((2, 5, 8))
    o = O.sdpa_gqa(q, kk, vv, 8 ** -0.5, False)
    for h in range(4):
        np.testing.assert_allclose(o[h], np.broadcast_to(vv[h // 2].mean(0), (3, 8)), rtol=1e-12)


def test_sdpa_fp16_p_closed_forms():
    """attention_fp16_p (fp16 P into P.V, the denominator the sum of those fp16 values): one
    key gives its value row; identical keys give the mean of V (every p = 1 exactly); against
    the default softmax the output moves only by P's fp16 rounding (relative 2^-11)."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 3, 128))
    k = rng.standard_normal((2, 1, 128))
    v = rng.standard_normal((2, 1, 128))
    with O.attention_fp16_p():
        out = O.sdpa_gqa(q, k, v, 128 ** -0.5, False)
    np.testing.assert_allclose(out, np.repeat(v, 2, axis=0).repeat(3, axis=1), rtol=1e-15)
    k2 = np.repeat(rng.standard_normal((2, 1, 128)), 7, axis=1)
    v2 = rng.standard_normal((2, 7, 128))
    with O.attention_fp16_p():
        out2 = O.sdpa_gqa(q, k2, v2, 128 ** -0.5, False)
    np.testing.assert_allclose(out2[0, 0], v2[0].mean(axis=0), rtol=1e-13)
    k3, v3 = rng.standard_normal((2, 50, 128)), rng.standard_normal((2, 50, 128))
    ref = O.sdpa_gqa(q, k3, v3, 128 ** -0.5, False)
    with O.attention_fp16_p():
        got = O.sdpa_gqa(q, k3, v3, 128 ** -0.5, False)
    assert 0 < np.abs(got - ref).max() < 2e-3


def test_sdpa_gqa_mapping_onehot():
    # V of kv head g is the constant g: output of query head h must be h // rep.
    NH, NKV, L, D = 8, 2, 5, 4
    rng = np.random.default_rng(8)
    q = rng.standard_normal((NH, 3, D))
    k = rng.standard_normal((NKV, L, D))
    v = np.stack([np.full((L, D), float(g)) for g in range(NKV)])
    o = O.sdpa_gqa(q, k, v, 0.5, False)
    for h in range(NH):
        np.testing.assert_allclose(o[h], h // (NH // NKV), atol=1e-12)


def test_sdpa_matches_torch():
    rng = np.random.default_rng(9)
    NH, NKV, Lq, L, D = 6, 2, 5, 11, 16
    q = rng.standard_normal((NH, Lq, D))
    k = rng.standard_normal((NKV, L, D))
    v = rng.standard_normal((NKV, L, D))
    tk = torch.from_numpy(k).repeat_interleave(NH // NKV, dim=0)
    tv = torch.from_numpy(v).repeat_interleave(NH // NKV, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q)[None], tk[None],
                                                           tv[None], scale=D ** -0.5)[0]
    np.testing.assert_allclose(O.sdpa_gqa(q, k, v, D ** -0.5, False), ref.numpy(), rtol=1e-10)


# ---------------------------------------------------------------------------
# Linear / MLP / lm_head
# ---------------------------------------------------------------------------

def test_linear_w8_exact_integer_and_onehot():
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((12, 20)) * 0.02).astype(np.float32)
    q, s = O.quantize_w8(w)
    x = rng.integers(-3, 4, size=(3, 20)).astype(np.float64)
    exact = np.array([[sum(int(x[m, k]) * int(q[n, k]) for k in range(20)) for n in range(12)]
                      for m in range(3)], dtype=np.float64) * s.astype(np.float64)
    np.testing.assert_array_equal(O.linear_w8(x, (q, s), False), exact)
    e = np.zeros((1, 20))
    e[0, 7] = 1.0
    np.testing.assert_array_equal(O.linear_w8(e, (q, s), False)[0],
                                  q[:, 7].astype(np.float64) * s.astype(np.float64))


def test_accumulation_split_orders():
    """accumulation_split(n) sums a reduction over n ordered contiguous ranges: exact
    integer sums are unchanged at every n, the fp32 result is the ordered sum of the range
    products computed by hand, the default (and the state after the context) is one plain
    matmul, and a ragged n (K not a multiple of n) still covers every k once."""
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((12, 23)) * 0.02).astype(np.float32)
    q, s = O.quantize_w8(w)
    x = rng.integers(-3, 4, size=(3, 23)).astype(np.float64)
    base = O.linear_w8(x, (q, s), False)
    for n in (2, 3, 4, 8):
        with O.accumulation_split(n):
            np.testing.assert_array_equal(O.linear_w8(x, (q, s), False), base)
    a = rng.standard_normal((5, 23)).astype(np.float32)
    b = rng.standard_normal((23, 7)).astype(np.float32)
    with O.accumulation_split(3):
        got = O._mm(a, b)
    want = ((a[:, 0:7] @ b[0:7]) + (a[:, 7:15] @ b[7:15])) + (a[:, 15:23] @ b[15:23])
    np.testing.assert_array_equal(got, want)
    np.testing.assert_allclose(got, a.astype(np.float64) @ b.astype(np.float64), rtol=1e-5,
                               atol=1e-5)
    np.testing.assert_array_equal(O._mm(a, b), a @ b)
    with O.accumulation_split(4):
        with O.accumulation_split(2):
            assert O._SPLIT[0] == 2
        assert O._SPLIT[0] == 4
    assert O._SPLIT[0] == 1


def test_mlp_zero_and_bruteforce():
    cfg = small_cfg()
    rng = np.random.default_rng(11)
    lw = {p: O.quantize_w8((rng.standard_normal(shp) * 0.1).astype(np.float32))
          for p, shp in [("gate_proj", (24, 16)), ("up_proj", (24, 16)), ("down_proj", (16, 24))]}
    np.testing.assert_array_equal(O.mlp(np.zeros((2, 16)), lw, False), 0.0)
    x = rng.standard_normal((2, 16))
    Wg, Wu, Wd = (O.dequantize_w8(*lw[p]) for p in ("gate_proj", "up_proj", "down_proj"))
    out = np.zeros((2, 16))
    for m in range(2):
        for n in range(16):
            acc = 0.0
            for f in range(24):
                g = sum(x[m, k] * Wg[f, k] for k in range(16))
                u = sum(x[m, k] * Wu[f, k] for k in range(16))
                acc += (g / (1 + math.exp(-g))) * u * Wd[n, f]
            out[m, n] = acc
    np.testing.assert_allclose(O.mlp(x, lw, False), out, rtol=1e-10, atol=1e-14)


def test_lm_head_argmax_onehot_planted_ties():
    V, H = 50, 8
    rng = np.random.default_rng(12)
    w = rng.standard_normal((V, H))
    h = np.zeros((1, H))
    h[0, 3] = 1.0
    logits, ids = O.lm_head_argmax(h, w)
    np.testing.assert_array_equal(logits[0], w[:, 3])
    assert ids[0] == int(np.argmax(w[:, 3]))
    w2 = np.zeros((V, H))
    w2[17, 0] = 5.0
    w2[33, 0] = 5.0   # tie -> lowest index
    w2[40, 0] = 4.9
    _, ids = O.lm_head_argmax(np.eye(1, H), w2)
    assert ids[0] == 17


# ---------------------------------------------------------------------------
# Whole forward: brute force on a tiny model, torch cross-check, invariants
# ---------------------------------------------------------------------------

def _tiny_weights(cfg, seed=0, nf=2):
    from mirror_sd_amd.synth import make_weights_numpy
    t = make_weights_numpy(cfg, seed=seed, n_feat=nf)
    # make the gains non-trivial so a dropped gain fails
    rng = np.random.default_rng(99)
    for k in list(t):
        if k.endswith("norm.weight"):
            t[k] = (1.0 + 0.3 * rng.standard_normal(t[k].shape)).astype(np.float16)
    # scale projections up so attention is not uniform
    for k in list(t):
        if t[k].dtype == np.float32:
            t[k] = t[k] * np.float32(20)
    return O.OracleWeights(cfg, t)


def _bruteforce_forward(W, noise, th):
    """Element-loop restatement of dflash.py:384-403, written independently."""
    cfg = W.cfg
    H, NH, NKV, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps

    def norm(vec, g):
        r = 1.0 / math.sqrt(sum(t * t for t in vec) / len(vec) + eps)
        return [vec[i] * r * float(g[i]) for i in range(len(vec))]

    def lin(vec, qs):
        q, s = qs
        return [float(s[n]) * sum(vec[k] * int(q[n, k]) for k in range(len(vec)))
                for n in range(q.shape[0])]

    def rope(vec, pos):
        half = D // 2
        out = [0.0] * D
        for j in range(half):
            a = pos * cfg.rope_theta ** (-2.0 * j / D)
            out[j] = vec[j] * math.cos(a) - vec[j + half] * math.sin(a)
            out[j + half] = vec[j + half] * math.cos(a) + vec[j] * math.sin(a)
        return out

    fcw = W.fc.astype(np.float64)
    ctx = []
    for row in th.astype(np.float64):
        f = [sum(row[k] * fcw[n, k] for k in range(row.shape[0])) for n in range(H)]
        ctx.append(norm(f, W.hidden_norm))
    C, B = len(ctx), noise.shape[0]
    x = [list(map(float, r)) for r in noise]
    for lw in W.layers:
        h = [norm(r, lw["input_layernorm"]) for r in x]
        kv_rows = ctx + h
        qv = [lin(r, lw["q_proj"]) for r in h]
        kv = [lin(r, lw["k_proj"]) for r in kv_rows]
        vv = [lin(r, lw["v_proj"]) for r in kv_rows]
        att = [[0.0] * (NH * D) for _ in range(B)]
        for hh in range(NH):
            g = hh // (NH // NKV)
            keys = [rope(norm(kv[j][g * D:(g + 1) * D], lw["k_norm"]), j) for j in range(C + B)]
            vals = [vv[j][g * D:(g + 1) * D] for j in range(C + B)]
            for i in range(B):
                qq = rope(norm(qv[i][hh * D:(hh + 1) * D], lw["q_norm"]), C + i)
                sc = [sum(qq[d] * kk[d] for d in range(D)) / math.sqrt(D) for kk in keys]
                mx_ = max(sc)
                e = [math.exp(t - mx_) for t in sc]
                z = sum(e)
                for d in range(D):
                    att[i][hh * D + d] = sum(e[j] * vals[j][d] for j in range(C + B)) / z
        o = [lin(r, lw["o_proj"]) for r in att]
        x = [[x[i][n] + o[i][n] for n in range(H)] for i in range(B)]
        h2 = [norm(r, lw["post_attention_layernorm"]) for r in x]
        gg = [lin(r, lw["gate_proj"]) for r in h2]
        uu = [lin(r, lw["up_proj"]) for r in h2]
        m = [[gg[i][f] / (1 + math.exp(-gg[i][f])) * uu[i][f] for f in range(len(gg[i]))]
             for i in range(B)]
        d = [lin(r, lw["down_proj"]) for r in m]
        x = [[x[i][n] + d[i][n] for n in range(H)] for i in range(B)]
    return np.array([norm(r, W.norm) for r in x])


def test_forward_bruteforce_tiny():
    cfg = small_cfg()
    W = _tiny_weights(cfg)
    rng = np.random.default_rng(13)
    noise = rng.standard_normal((4, 16)).astype(np.float16)
    th = rng.standard_normal((3, 32)).astype(np.float16)
    ref = _bruteforce_forward(W, noise, th)
    got = O.draft_forward(W, noise, th, fp16=False)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-11)


def _torch_forward(W, noise, th):
    """Library cross-check: the same forward in torch float64 ops (F.rms_norm,
    complex-multiplication RoPE, F.scaled_dot_product_attention)."""
    F = torch.nn.functional
    cfg = W.cfg
    H, NH, NKV, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps
    T = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float64))
    deq = lambda qs: T(O.dequantize_w8(*qs))

    def rope(x, pos):  # x [L, heads, D]
        z = torch.complex(x[..., :D // 2], x[..., D // 2:])
        inv = T(cfg.rope_theta ** (-2.0 * np.arange(D // 2) / D))
        rot = torch.polar(torch.ones_like(inv)[None, :].expand(len(pos), -1),
                          T(pos)[:, None] * inv[None, :])
        zr = z * rot[:, None, :]
        return torch.cat([zr.real, zr.imag], dim=-1)

    ctx = F.rms_norm(T(th) @ T(W.fc).T, (H,), T(W.hidden_norm), eps)
    x = T(noise)
    C, B = ctx.shape[0], x.shape[0]
    for lw in W.layers:
        h = F.rms_norm(x, (H,), T(lw["input_layernorm"]), eps)
        kvin = torch.cat([ctx, h])
        q = F.rms_norm((h @ deq(lw["q_proj"]).T).view(B, NH, D), (D,), T(lw["q_norm"]), eps)
        k = F.rms_norm((kvin @ deq(lw["k_proj"]).T).view(C + B, NKV, D), (D,), T(lw["k_norm"]), eps)
        v = (kvin @ deq(lw["v_proj"]).T).view(C + B, NKV, D)
        q = rope(q, np.arange(C, C + B))
        k = rope(k, np.arange(C + B))
        o = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                           scale=D ** -0.5, enable_gqa=True)
        x = x + o.transpose(0, 1).reshape(B, NH * D) @ deq(lw["o_proj"]).T
        h2 = F.rms_norm(x, (H,), T(lw["post_attention_layernorm"]), eps)
        x = x + (F.silu(h2 @ deq(lw["gate_proj"]).T) * (h2 @ deq(lw["up_proj"]).T)) @ deq(lw["down_proj"]).T
    return F.rms_norm(x, (H,), T(W.norm), eps).numpy()


def test_forward_matches_torch_library():
    cfg = small_cfg(H=64, NH=8, NKV=2, D=16, F=96, L=3)
    W = _tiny_weights(cfg)
    rng = np.random.default_rng(14)
    noise = rng.standard_normal((5, 64)).astype(np.float16)
    th = rng.standard_normal((7, 128)).astype(np.float16)
    np.testing.assert_allclose(O.draft_forward(W, noise, th, fp16=False),
                               _torch_forward(W, noise, th), rtol=1e-9, atol=1e-10)


def test_fp16_mode_close_to_ideal():
    cfg = small_cfg(H=64, NH=8, NKV=2, D=16, F=96, L=3)
    W = _tiny_weights(cfg)
    rng = np.random.default_rng(15)
    noise = rng.standard_normal((5, 64)).astype(np.float16)
    th = rng.standard_normal((7, 128)).astype(np.float16)
    a = O.draft_forward(W, noise, th, fp16=False)
    b = O.draft_forward(W, noise, th, fp16=True)
    assert np.all(b == b.astype(np.float16))            # every output is an fp16 value
    cos = (a * b).sum() / np.linalg.norm(a) / np.linalg.norm(b)
    assert cos > 0.9995 and np.abs(a - b).max() < 3e-2


def test_cache_two_step_equals_single_pass():
    """Ingesting context in two calls through the cache (with trim of the block)
    gives the same block output as one cache-less call over the whole context:
    context rows never pass through layers and positions are absolute."""
    cfg = small_cfg(H=32, NH=4, NKV=2, D=8, F=48, L=2)
    W = _tiny_weights(cfg)
    rng = np.random.default_rng(16)
    th = rng.standard_normal((9, 64)).astype(np.float16)
    noise = rng.standard_normal((4, 32)).astype(np.float16)
    ref = O.draft_forward(W, noise, th, fp16=False)
    caches = [O.OracleKVCache() for _ in range(cfg.num_hidden_layers)]
    # step 1: first 5 context rows with a throwaway block, then trim the block
    O.draft_forward(W, noise, th[:5], cache=caches, fp16=False)
    for c in caches:
        c.trim(4)
    assert caches[0].offset == 5 and caches[0].keys.shape[1] == 5
    out = O.draft_forward(W, noise, th[5:], cache=caches, fp16=False)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    assert caches[0].offset == 9 + 4


def test_context_rows_independent_of_block():
    """K/V of context rows depend only on the fused context: changing the block
    input changes the outputs but not the cached context K/V."""
    cfg = small_cfg()
    W = _tiny_weights(cfg)
    rng = np.random.default_rng(17)
    th = rng.standard_normal((3, 32)).astype(np.float16)
    c1 = [O.OracleKVCache() for _ in range(2)]
    c2 = [O.OracleKVCache() for _ in range(2)]
    O.draft_forward(W, rng.standard_normal((4, 16)).astype(np.float16), th, cache=c1, fp16=False)
    O.draft_forward(W, rng.standard_normal((4, 16)).astype(np.float16), th, cache=c2, fp16=False)
    for a, b in zip(c1, c2):
        np.testing.assert_array_equal(a.keys[:, :3], b.keys[:, :3])
        np.testing.assert_array_equal(a.values[:, :3], b.values[:, :3])
        assert not np.allclose(a.keys[:, 3:], b.keys[:, 3:])


def test_cache_window_eviction():
    c = O.OracleKVCache(sink_size=2, window_size=3)
    k = np.arange(8, dtype=np.float64).reshape(1, 8, 1)
    c.update_and_fetch(k[:, :4], k[:, :4])
    c.update_and_fetch(k[:, 4:], k[:, 4:])
    assert c.keys[0, :, 0].tolist() == [0, 1, 5, 6, 7] and c.offset == 8
    c.trim(2)
    assert c.keys[0, :, 0].tolist() == [0, 1, 5] and c.offset == 6


# ---------------------------------------------------------------------------
# Soft anchor (generate.py:1419-1437)
# ---------------------------------------------------------------------------

def _emb(V=300, H=32, seed=0):
    return np.random.default_rng(seed).normal(0, 0.02, (V, H)).astype(np.float16)


def test_soft_anchor_top1_is_argmax_row():
    E = _emb()
    lg = np.random.default_rng(1).normal(0, 3, E.shape[0]).astype(np.float32)
    np.testing.assert_array_equal(O.soft_anchor(E, lg, top_k=1), E[int(np.argmax(lg))])


def test_soft_anchor_dominant_logit_gives_its_row():
    E = _emb()
    lg = np.random.default_rng(2).normal(0, 1, E.shape[0]).astype(np.float32)
    lg[123] = 200.0   # exp(x - 200) underflows to 0 for every other selected logit
    np.testing.assert_array_equal(O.soft_anchor(E, lg), E[123])


def test_soft_anchor_equal_logits_give_mean_row():
    E = _emb()
    lg = np.full(E.shape[0], -5.0, dtype=np.float32)
    top = [7, 40, 41, 99, 150, 151, 200, 299]
    lg[top] = 2.5
    want = E[top].astype(np.float64).mean(0)
    got = O.soft_anchor(E, lg).astype(np.float64)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=2e-3)


def test_soft_anchor_two_rows_closed_form():
    """Logits differing by ln 3 (the rest at -inf) weigh the rows 3/4 and 1/4."""
    E = _emb()
    lg = np.full(E.shape[0], -np.inf, dtype=np.float32)
    lg[10], lg[20] = 1.0 + math.log(3.0), 1.0
    want = 0.75 * E[10].astype(np.float64) + 0.25 * E[20].astype(np.float64)
    np.testing.assert_allclose(O.soft_anchor(E, lg).astype(np.float64), want, atol=2e-5)


def test_soft_anchor_selection_and_weights_against_library():
    """The selected ids are the top-k by np.argpartition; the weights are scipy's softmax."""
    from scipy.special import softmax
    E = _emb(V=1000, H=16)
    lg = np.random.default_rng(3).normal(0, 2, 1000).astype(np.float32)
    top = np.argpartition(-lg, 8)[:8]
    w = softmax(lg[top].astype(np.float64))
    want = (w[:, None] * E[top].astype(np.float64)).sum(0)
    np.testing.assert_allclose(O.soft_anchor(E, lg).astype(np.float64), want, atol=1e-5,
                               rtol=2e-3)


def test_soft_anchor_ties_pick_lowest_ids_and_skip_nan():
    E = _emb()
    lg = np.zeros(E.shape[0], dtype=np.float32)
    lg[[5, 9, 250]] = np.nan
    # every number ties: the 3 lowest non-NaN ids are 0, 1, 2
    want = E[[0, 1, 2]].astype(np.float64).mean(0)
    np.testing.assert_allclose(O.soft_anchor(E, lg, top_k=3).astype(np.float64), want,
                               atol=1e-5, rtol=2e-3)
    lg2 = np.full(E.shape[0], np.nan, dtype=np.float32)
    lg2[17] = -3.0
    np.testing.assert_array_equal(O.soft_anchor(E, lg2), E[17])


def test_embed_block_rows():
    E = _emb()
    ids = np.array([3, 299, 299, 0])
    np.testing.assert_array_equal(O.embed_block(E, ids), E[ids])
    lg = np.zeros(E.shape[0], dtype=np.float32)
    lg[42] = 300.0
    out = O.embed_block(E, ids, lg)
    np.testing.assert_array_equal(out[0], E[42])
    np.testing.assert_array_equal(out[1:], E[ids[1:]])
