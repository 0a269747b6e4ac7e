"""Run the reference's own scripts on this library, unchanged.

Every Python caller of the reference puts its own checkout first on ``sys.path`` before it
imports the kernels (``sys.path.insert(0, ROOT)``: test_mla.py:9, scripts/check_mla.py:14,
scripts/mla_prof.py:19, scripts/scan_ns.py:17, scripts/bench_mla_heads.py:29), so a path
entry can never make ``import mla_decode`` pick this repository's module.  An import hook can:
a finder on ``sys.meta_path`` is asked before any ``sys.path`` entry, whatever order the caller
gives them.

    python -m mlc_decode_amd.dropin /path/to/reference/test_mla.py [args...]

runs the script as ``__main__`` with ``mla_decode`` and ``baseline_mla`` resolved to the
drop-in modules at this repository's root.  Inside a process, ``install_import_hook()`` does
the same before the caller's imports.
"""
from __future__ import annotations

import importlib.abc
import importlib.util
import os
import runpy
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# module name -> the file of this repository that replaces it
MODULES = {
    "mla_decode": os.path.join(REPO, "mla_decode.py"),
    "baseline_mla": os.path.join(REPO, "baseline_mla.py"),
}


class _DropInFinder(importlib.abc.MetaPathFinder):
    """Resolves the reference's kernel modules to this repository's files."""

    def find_spec(self, fullname, path=None, target=None):
        file = MODULES.get(fullname)
        if file is None:
            return None
        return importlib.util.spec_from_file_location(fullname, file)


_FINDER = _DropInFinder()


def install_import_hook() -> None:
    """Make ``import mla_decode`` / ``import baseline_mla`` load this repository's modules,
    whatever ``sys.path`` holds.  Idempotent; modules already imported under those names are
    dropped so the next import resolves afresh."""
    if _FINDER not in sys.meta_path:
        sys.meta_path.insert(0, _FINDER)
    if REPO not in sys.path:
        sys.path.append(REPO)  # for ``mlc_decode_amd`` itself
    for name, file in MODULES.items():
        mod = sys.modules.get(name)
        if mod is not None and os.path.abspath(getattr(mod, "__file__", "") or "") != file:
            del sys.modules[name]


def main(argv=None) -> None:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] in ("-h", "--help"):
        print(__doc__)
        raise SystemExit(0 if argv else 2)
    script = os.path.abspath(argv[0])
    install_import_hook()
    sys.argv = [script] + argv[1:]
    # the script sees its own directory first, as when started as `python script.py`
    sys.path.insert(0, os.path.dirname(script))
    runpy.run_path(script, run_name="__main__")


if __name__ == "__main__":
    main()
