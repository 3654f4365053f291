import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mirror-sd_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _ensure_built():
    lib = os.path.join(ROOT, "mirror-sd_amd", "mirror_sd_amd", "libdflash_hip.so")
    if not os.path.exists(lib):
        import importlib.util
        spec = importlib.util.spec_from_file_location("dfl_build", os.path.join(ROOT, "mirror-sd_amd", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build(verbose=False)


_ensure_built()


def pytest_terminal_summary(terminalreporter):
    """Session total of the draft-token agreement recorded by parity_util.check_argmax."""
    try:
        from parity_util import ARGMAX_TOTALS
    except ImportError:
        return
    n = ARGMAX_TOTALS["rows"]
    if n:
        a = ARGMAX_TOTALS["agree"]
        terminalreporter.write_line(
            f"argmax agreement over {len(ARGMAX_TOTALS['cases'])} checks: {a}/{n} = {a / n:.4f} "
            f"(exempt: {ARGMAX_TOTALS['undecided']} oracle-undecided, {ARGMAX_TOTALS['noise']} "
            f"listed unbacked)")
        for what, n_agree, rows, n_und, n_noise in ARGMAX_TOTALS["cases"]:
            if n_agree < rows:
                terminalreporter.write_line(
                    f"  {what}: {n_agree}/{rows} (exempt {n_und} oracle-undecided, "
                    f"{n_noise} listed unbacked)")
