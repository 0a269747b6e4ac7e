"""A caller of the reference puts its own checkout first on sys.path before importing the
kernels; through ``mlc_decode_amd.dropin`` it still gets this repository's modules.  Runs on
the CPU: imports and the host-side split rule only, no kernel launch."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# A stand-in for a reference script (written here): it inserts its own directory first, as the
# reference's callers do, then imports the names they import.
CALLER = """
import os, sys
ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
from mla_decode import (_get_kernel, _split_plan, build_kernel_from_config, flashattn_frag_q,
                        flashattn_shared_q, mla_autotune_configs, run_kernel)
from baseline_mla import _get_kernel as baseline_kernel, ref_program
import baseline_mla, mla_decode
print("mla_decode from", mla_decode.__file__)
print("baseline_mla from", baseline_mla.__file__)
print("split plan", _split_plan(4096, 4, 64, False))
"""
# What the caller's own checkout would give it: the reference modules import TileLang.
DECOY = 'raise ImportError("reference module: needs tilelang")\n'


def _write_root(tmp_path):
    (tmp_path / "caller.py").write_text(CALLER)
    (tmp_path / "mla_decode.py").write_text(DECOY)
    (tmp_path / "baseline_mla.py").write_text(DECOY)
    return str(tmp_path / "caller.py")


def test_caller_alone_imports_its_own_checkout(tmp_path):
    caller = _write_root(tmp_path)
    env = dict(os.environ, PYTHONPATH=REPO)  # a path entry cannot win: the caller goes first
    r = subprocess.run([sys.executable, caller], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode != 0 and "needs tilelang" in r.stderr


def test_dropin_runner_resolves_this_repository(tmp_path):
    caller = _write_root(tmp_path)
    r = subprocess.run([sys.executable, "-m", "mlc_decode_amd.dropin", caller, "--flag"],
                       capture_output=True, text=True, cwd=REPO, timeout=300)
    assert r.returncode == 0, r.stderr
    assert f"mla_decode from {os.path.join(REPO, 'mla_decode.py')}" in r.stdout
    assert f"baseline_mla from {os.path.join(REPO, 'baseline_mla.py')}" in r.stdout
    assert "split plan (4, 16, 0)" in r.stdout


def test_import_hook_in_process(tmp_path, monkeypatch):
    _write_root(tmp_path)
    monkeypatch.syspath_prepend(str(tmp_path))
    for name in ("mla_decode", "baseline_mla"):
        monkeypatch.delitem(sys.modules, name, raising=False)
    from mlc_decode_amd import dropin
    dropin.install_import_hook()
    try:
        import mla_decode
        assert mla_decode.__file__ == os.path.join(REPO, "mla_decode.py")
    finally:
        sys.meta_path.remove(dropin._FINDER)
