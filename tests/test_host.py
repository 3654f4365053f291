"""Host-side tests that need no GPU: the C ABI library loads and exports every
symbol the header declares, argument validation runs before any device work,
and the config / synthetic-input helpers behave like the reference's."""

import ctypes
import os
import re

import numpy as np
import pytest

from mirror_sd_amd import _lib
from mirror_sd_amd.config import DFlashConfig, build_target_layer_ids, extract_context_feature, workload
from mirror_sd_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dflash_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dfl_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    syms = _declared_symbols()
    assert len(syms) >= 15
    lib = _lib.load()
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in dflash_hip.h but not exported"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(syms)


def test_no_kernel_spills():
    """Every kernel of the last build fits in its registers: no scratch memory (register
    spills) and no dynamic stack, from the compiler's resource-usage record of the build."""
    import json
    path = os.path.join(ROOT, "mirror-sd_amd", "_build", "kernel_resources.json")
    if not os.path.exists(path):
        pytest.skip("no resource record: the library was not built by mirror-sd_amd/build.py here")
    usage = json.load(open(path))
    assert sum("block_attn_kernel" in k for k in usage) >= 4 and len(usage) >= 50
    spills = {k: v["ScratchSize [bytes/lane]"] for k, v in usage.items()
              if v["ScratchSize [bytes/lane]"] or v["VGPRs Spill"] or v["Dynamic Stack"] != "False"}
    assert not spills, f"kernels using scratch (bytes per lane): {spills}"


def _cfg(**over):
    c = dict(hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, n_layers=2,
             n_target_feat=5, vocab=1024, max_block=16, max_ctx=64, rms_eps=1e-6,
             rope_theta=1e6)
    c.update(over)
    return _lib.DflConfig(**c)


@pytest.mark.parametrize("over,needle", [
    (dict(head_dim=64), "head_dim"),
    (dict(hidden=100), "hidden"),
    (dict(n_heads=5, n_kv_heads=2), "n_heads"),
    (dict(intermediate=100), "intermediate"),
    (dict(vocab=1000), "vocab"),
    (dict(max_block=0), "max_block"),
    (dict(max_block=1000), "max_block"),
    (dict(rms_eps=0.0), "rms_eps"),
    (dict(n_layers=0), "n_layers"),
])
def test_create_validates_config(over, needle):
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.dfl_create(ctypes.byref(_cfg(**over)), ctypes.byref(h))
    assert rc == _lib.DFL_EINVAL and not h.value
    assert needle in lib.dfl_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(rc, "dfl_create")


def test_null_context_errors():
    lib = _lib.load()
    assert lib.dfl_cache_trim(None, 1) == _lib.DFL_EINVAL
    assert lib.dfl_draft_block(None, None, None, 1, None, None, None, None, None) == _lib.DFL_EINVAL
    assert lib.dfl_quantize_w8(None, 1, 1, None, None, None) == _lib.DFL_EINVAL
    assert lib.dfl_create(None, None) == _lib.DFL_EINVAL
    assert "null" in lib.dfl_last_error().decode()


def test_noalloc_embed_block_validates_before_device_work():
    """dfl_embed_block_noalloc rejects bad arguments before it touches a device (these
    pointers are never dereferenced)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)   # 16-byte aligned, never read
    args = lambda **o: dict(dict(ids=fake, B=4, embed=fake, Vemb=1024, H=256, lg=None, dt=0,
                                 V=0, k=8, out=fake, err=fake), **o)
    call = lambda a: lib.dfl_embed_block_noalloc(a["ids"], a["B"], a["embed"], a["Vemb"], a["H"],
                                                 a["lg"], a["dt"], a["V"], a["k"], a["out"],
                                                 a["err"], None)
    for bad, needle in [(dict(ids=None), "null"), (dict(err=None), "null"), (dict(H=100), "H"),
                        (dict(embed=ctypes.c_void_p(4100)), "alignment"), (dict(B=0), "rows"),
                        (dict(lg=fake, dt=3, V=64), "logits_dtype"),
                        (dict(lg=fake, V=64, k=9), "top_k"), (dict(lg=fake, V=2048), "length")]:
        assert call(args(**bad)) == _lib.DFL_EINVAL, bad
        assert needle in lib.dfl_last_error().decode(), (bad, lib.dfl_last_error())


def test_launch_argument_checks(tmp_path):
    """The host-side checks of the kernel launch structs (dfl_check.h) refuse each kind of
    inconsistent argument: built with hipcc as a host program and run on the CPU."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = str(tmp_path / "check_args_host")
    csrc = os.path.join(ROOT, "mirror-sd_amd", "csrc")
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-std=c++17", "-O1", "-I", csrc,
                        os.path.join(ROOT, "tests", "check_args_host.hip"), "-o", exe],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


def test_launch_argument_checks_sanitized(tmp_path):
    """The same host program built with AddressSanitizer and UndefinedBehaviorSanitizer on its
    host code (the launch checks and the tile planner are host code): no out-of-bounds
    access, leak or undefined behaviour in any of the checks."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = str(tmp_path / "check_args_host_san")
    csrc = os.path.join(ROOT, "mirror-sd_amd", "csrc")
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-std=c++17", "-O1", "-g",
                        "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                        "-Xarch_host", "-fno-sanitize-recover=undefined",
                        "-Xarch_host", "-fno-omit-frame-pointer", "-I", csrc,
                        os.path.join(ROOT, "tests", "check_args_host.hip"), "-o", exe],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


def test_build_target_layer_ids():
    assert build_target_layer_ids(36, 5) == [1, 9, 17, 25, 33]
    assert build_target_layer_ids(36, 1) == [18]
    assert build_target_layer_ids(64, 5) == [1, 16, 31, 46, 61]
    assert build_target_layer_ids(35, 5) == [1, 9, 16, 24, 32]   # round(16.5) == 16 (half-even)


def test_from_dict_defaults_follow_reference():
    c = DFlashConfig.from_dict({})
    assert c.rope_theta == 10000.0 and c.mask_token_id == 151667 and c.num_key_value_heads == 2
    assert c.intermediate_size == 10944 and c.max_position_embeddings == 4096
    d = DFlashConfig()
    assert d.rope_theta == 1e6 and d.mask_token_id == 151669
    c = DFlashConfig.from_dict({"dflash_config": {"target_layer_ids": [2, 3], "block_size": 32,
                                                   "mask_token_id": 7}, "hidden_size": 5120})
    assert c.target_layer_ids == [2, 3] and c.block_size == 32 and c.mask_token_id == 7
    assert c.num_target_features == 2 and c.hidden_size == 5120


def test_extract_context_feature():
    hs = [np.full((1, 2, 3), i, dtype=np.float32) for i in range(6)]
    out = extract_context_feature(hs, [0, 2, 4])
    assert out.shape == (1, 2, 9) and list(out[0, 0, ::3]) == [1, 3, 5]
    out = extract_context_feature(hs[:3], [0, 2, 4])
    assert list(out[0, 0, ::3]) == [0, 1, 2]


def test_synth_deterministic_and_order_independent():
    cfg = workload("tiny").cfg
    a = synth.make_weights_numpy(cfg, seed=0)
    b = synth.make_weights_numpy(cfg, seed=0)
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])
    # a tensor generated on its own equals the same tensor generated among all others
    name = "layers.1.mlp.up_proj.weight"
    x = synth.np_normal(0, name, a[name].shape, 0.02)
    np.testing.assert_array_equal(x, a[name])
    c = synth.make_weights_numpy(cfg, seed=1)
    assert not np.array_equal(a["fc.weight"], c["fc.weight"])
    inp = synth.make_inputs_numpy(cfg, 8, 24, seed=0)
    assert inp["ids"][0] < cfg.vocab_size and np.all(inp["ids"][1:] == cfg.mask_token_id)
    assert inp["target_hidden"].shape == (24, 5 * 256) and inp["target_hidden"].dtype == np.float16


def test_workload_shapes():
    w = workload("dflash_27b")
    assert (w.cfg.hidden_size, w.cfg.num_attention_heads, w.cfg.num_key_value_heads,
            w.cfg.intermediate_size, w.block, w.ctx) == (5120, 40, 8, 17408, 32, 4096)
    assert workload("dflash_27b_ctx32768").ctx == 32768
    w = workload("qwen3_4b_layer")
    assert (w.cfg.hidden_size, w.cfg.intermediate_size, w.cfg.num_hidden_layers) == (2560, 9728, 1)


def test_bench_compiles_and_refuses_several_gpus():
    """bench.py parses (a subprocess compiles the whole file) and exits with a message for
    --gpus N > 1 (one GPU per box) before touching a GPU."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, r.stderr
    assert "one GPU" in r.stderr


def test_model_refuses_unimplemented_rope_scaling():
    """A rope_scaling type the library does not implement (yarn) is refused by the model
    itself, not only by the loader; default, linear and llama3 map to the library's RoPE
    types with mlx_lm's defaults for absent llama3 keys (initialize_rope, called at
    dflash.py:254-261)."""
    from mirror_sd_amd.dflash import DFlashDraftModel
    from mirror_sd_amd.config import rope_scaling_args, ROPE_DEFAULT, ROPE_LINEAR, ROPE_LLAMA3
    cfg = DFlashConfig.from_dict({"hidden_size": 256, "num_hidden_layers": 1,
                                  "rope_scaling": {"rope_type": "yarn", "factor": 4.0}})
    with pytest.raises(NotImplementedError):
        DFlashDraftModel(cfg, max_ctx=16)
    for rs, want in [(None, ROPE_DEFAULT), ({"rope_type": "default"}, ROPE_DEFAULT),
                     ({"type": "linear", "factor": 2.0}, ROPE_LINEAR)]:
        cfg = DFlashConfig.from_dict({"hidden_size": 256, **({"rope_scaling": rs} if rs else {})})
        assert rope_scaling_args(cfg)[0] == want
    cfg = DFlashConfig.from_dict({"rope_scaling": {"rope_type": "llama3", "factor": 8.0}})
    assert rope_scaling_args(cfg) == (ROPE_LLAMA3, 8.0, 1.0, 4.0, 8192)
    # "type" is read before "rope_type", as mlx_lm does
    cfg = DFlashConfig.from_dict({"rope_scaling": {"type": "llama3", "rope_type": "yarn",
                                                   "factor": 32.0, "low_freq_factor": 2.0,
                                                   "high_freq_factor": 8.0,
                                                   "original_max_position_embeddings": 4096}})
    assert rope_scaling_args(cfg) == (ROPE_LLAMA3, 32.0, 2.0, 8.0, 4096)


def test_host_ids_checked_device_ids_not_read_back():
    """Host token ids outside [0, V) raise at the call; the check never reads device ids back
    (the kernels flag those in the device error word instead)."""
    import torch
    from mirror_sd_amd.dflash import _check_ids
    with pytest.raises(ValueError):
        _check_ids([0, 5, 7], 7)
    with pytest.raises(ValueError):
        _check_ids(torch.tensor([-1, 2]), 7)
    t = _check_ids(np.array([[1, 2], [3, 4]], dtype=np.int64), 7, flat=False)
    assert t.dtype == torch.int32 and t.shape == (2, 2)


def test_rocprof_summary_trace_skips_warmup_blocks(tmp_path):
    """Trace mode of the profile summariser: the dispatches of the first N blocks (from
    the first block-start kernel to the start of block N + 1) are left out; dispatches
    before the first block (context ingest) and after the warmup are averaged."""
    from mirror_sd_amd import rocprof_summary as rs
    seq = [("ingest_k", 100)] + [(k, d) for b in range(4)
                                 for k, d in (("embed_norm_kernel", 10 + b), ("gemm_k", 50 + b))]
    path = tmp_path / "t_kernel_trace.csv"
    t, lines = 0, ["Kernel_Name,Start_Timestamp,End_Timestamp"]
    for name, dur in seq:
        lines.append(f"{name},{t},{t + dur}")
        t += dur + 5
    path.write_text("\n".join(lines) + "\n")
    st = rs.read_trace(str(path), 2, r"embed_norm")
    assert st == {"ingest_k": (1, 100.0), "embed_norm_kernel": (2, 12.0 + 13.0),
                  "gemm_k": (2, 52.0 + 53.0)}
    assert rs.read_trace(str(path), 0, r"embed_norm")["gemm_k"] == (4, 50.0 + 51 + 52 + 53)
    assert rs.read_trace(str(path), 9, r"embed_norm") == {"ingest_k": (1, 100.0)}
    # from the 3rd gemm_k dispatch on (blocks 2 and 3), nothing else skipped
    assert rs.read_trace(str(path), 0, r"embed_norm", r"gemm_k", 2) == {
        "embed_norm_kernel": (1, 13.0), "gemm_k": (2, 52.0 + 53.0)}
    # from the 2nd gemm_k on, up to the first embed_norm after it less one more dispatch:
    # gemm_k of blocks 1 and 2 and embed_norm of block 2 ... up to block 3's embed_norm
    assert rs.read_trace(str(path), 0, r"embed_norm", r"gemm_k", 1, r"embed_norm_kernel", 0) == {
        "gemm_k": (1, 51.0)}
    assert rs.read_trace(str(path), 0, r"embed_norm", r"gemm_k", 0, r"gemm_k_none", 0) == {
        "gemm_k": (4, 50.0 + 51 + 52 + 53), "embed_norm_kernel": (3, 11.0 + 12 + 13)}
    assert rs.read_trace(str(path), 0, r"embed_norm", r"ingest_k", 0, r"gemm_k", 1) == {
        "ingest_k": (1, 100.0)}


def test_argmax_agreement_rule():
    """parity_util.check_argmax: a GPU id that differs from the oracle's fp32 run passes only
    if another accumulation run of the oracle picked it (any row of alt_ids) and the check's
    committed budget of such rows is not exceeded, or if the row is listed with that id in
    KNOWN_UNBACKED; a runner-up inside any gap, however small, raises otherwise.  The exact
    ids must be the logits' argmax."""
    import copy
    import parity_util as P
    saved = copy.deepcopy(P.ARGMAX_TOTALS)   # synthetic rows stay out of the session totals
    budgets, known = dict(P.EXEMPT_BUDGET), dict(P.KNOWN_UNBACKED)
    try:
        P.EXEMPT_BUDGET["alt run"] = 1
        P.EXEMPT_BUDGET["alt run, two rows"] = 1
        P.KNOWN_UNBACKED[("listed", 4)] = 1 + 4 % 16
        _argmax_rule_cases(P)
    finally:
        P.ARGMAX_TOTALS.clear()
        P.ARGMAX_TOTALS.update(saved)
        P.EXEMPT_BUDGET.clear()
        P.EXEMPT_BUDGET.update(budgets)
        P.KNOWN_UNBACKED.clear()
        P.KNOWN_UNBACKED.update(known)


def _argmax_rule_cases(P):
    rows, V = 6, 16
    ref = np.arange(rows) % V
    lg = np.zeros((rows, V))
    lg[np.arange(rows), ref] = 1.0
    ti = np.stack([ref, (ref + 1) % V], 1)
    tv = np.take_along_axis(lg, ti, 1).copy()
    tv[:, 1] = 0.5
    ids = ref.copy()
    # row 2: the GPU picks id 9, which the oracle's second alternative run also picked
    ids[2] = 9
    lg[2] = 0.0
    lg[2, 9] = 1.0
    alts = np.stack([ref, ref.copy()])
    alts[1, 2] = 9
    assert P.check_argmax(ids, lg, ref, alts, "alt run", ti, tv, 5.0) == (5, 6, 1)
    with pytest.raises(AssertionError):   # no other run picked it
        P.check_argmax(ids, lg, ref, alts[:1], "alt run", ti, tv, 5.0)
    with pytest.raises(AssertionError):   # an unlisted check has no budget
        P.check_argmax(ids, lg, ref, alts, "no budget", ti, tv, 5.0)
    # two backed rows against a budget of one
    ids3, lg3, alts3 = ids.copy(), lg.copy(), alts.copy()
    ids3[3] = 11
    lg3[3] = 0.0
    lg3[3, 11] = 1.0
    alts3[0, 3] = 11
    with pytest.raises(AssertionError):
        P.check_argmax(ids3, lg3, ref, alts3, "alt run, two rows", ti, tv, 5.0)
    # row 4: the runner-up with a gap of 1e-9, backed by no run: fails unless listed
    ids2 = ref.copy()
    ids2[4] = ti[4, 1]
    lg2 = lg.copy()
    lg2[2] = 0.0
    lg2[2, ref[2]] = 1.0
    lg2[4] = 0.0
    lg2[4, ti[4, 1]] = 1.0
    tv2 = tv.copy()
    tv2[4] = [1.0, 1.0 - 1e-9]
    with pytest.raises(AssertionError):
        P.check_argmax(ids2, lg2, ref, ref, "strict", ti, tv2, 5.0)
    assert P.check_argmax(ids2, lg2, ref, ref, "listed", ti, tv2, 5.0)[2] == 1
    ids4, lg4 = ids2.copy(), lg2.copy()   # a listed row with another id fails
    ids4[4] = 7
    lg4[4] = 0.0
    lg4[4, 7] = 1.0
    with pytest.raises(AssertionError):
        P.check_argmax(ids4, lg4, ref, ref, "listed", ti, tv2, 5.0)
    with pytest.raises(AssertionError):   # ids must be the argmax of the logits
        P.check_argmax(ids, lg2, ref, alts, "not argmax", ti, tv, 5.0)


def test_rocprof_summary_groups_match_the_built_kernels():
    """The profile summariser's kernel groups match the stream-K instantiations the build
    records (names demangled as a kernel trace shows them), each in the intended group:
    the projection row takes qkv, o / down and gate|up and nothing else."""
    import json
    import shutil
    import subprocess
    from mirror_sd_amd import rocprof_summary as rs
    groups = dict(rs.GROUPS)
    expect = {
        "void dfl::gsk_gemm_kernel<0, 5, true, 4, false>(dfl::StreamArgs)": "qkv (",
        "void dfl::gsk_gemm_kernel<0, 4, false, 4, false>(dfl::StreamArgs)": "o / down",
        "void dfl::gsk_gemm_kernel<0, 1, true, 4, false>(dfl::StreamArgs)": "gate|up",
        "void dfl::gsk_dyn_kernel<1, 2, true, 4>(dfl::StreamArgs)": "lm_head",
        "void dfl::gsk_gemm_kernel<1, 4, false, 4, true>(dfl::StreamArgs)": "read in place",
        "void dfl::gsk_gemm_kernel<1, 4, false, 4, false>(dfl::StreamArgs)": "gathered",
        "void dfl::gsk_gemm_kernel<0, 3, true, 4, false>(dfl::StreamArgs)": "K|V, all layers",
    }
    for name, label in expect.items():
        hits = [g for g, rx in groups.items() if re.search(rx, name) and g != "proj_gemm_w8a16"]
        assert len(hits) == 1 and label in hits[0], (name, hits)
        in_proj = bool(re.search(groups["proj_gemm_w8a16"], name))
        assert in_proj == (label in ("qkv (", "o / down", "gate|up")), name
    res = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "mirror-sd_amd", "_build", "kernel_resources.json")
    if not (os.path.exists(res) and shutil.which("c++filt")):
        pytest.skip("no build record or c++filt")
    with open(res) as f:
        mangled = [k for k in json.load(f) if "gsk_" in k]
    out = subprocess.run(["c++filt"], input="\n".join(mangled), capture_output=True, text=True,
                         check=True).stdout.split("\n")
    built = {n.strip() for n in out if n.strip()}
    assert set(expect) <= built, sorted(set(expect) - built)
