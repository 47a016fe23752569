"""Run one of the reference's harness scripts against this build, unchanged.

    python <repo>/kernelgen-challenge_amd/run_reference.py test_correctness.py [args]
    python <repo>/kernelgen-challenge_amd/run_reference.py -m pytest [pytest args]

Run it from inside a track directory (``track-01/``, ``track-02/`` or
``track-03/`` of the reference). The harness scripts import ``submission``,
``workloads`` and ``reference.reference`` by bare module name
(track-01/test_correctness.py:12-14, track-01/bench.py:11-13,
track-01/profile.py:9-10, track-02/test_correctness.py:12-14,
track-03/test_correctness.py:9-11). Launched the usual way
(``python test_correctness.py``, ``python -m pytest``) the script's own
directory (or the current one) comes first on ``sys.path``, so ``submission``
resolves to the track's own Triton file, whatever ``PYTHONPATH`` says.

This launcher puts this package's directory first and the script's directory
(for ``-m``: the current directory) second, then runs the script as
``__main__`` in the same process, the way ``python script.py`` would:
``submission`` resolves here and ``workloads`` / ``reference`` still resolve
to the track, because the package holds no module of those names.

With ``-m pytest`` it adds ``--import-mode=append`` unless the arguments
choose an import mode: pytest's default mode (``prepend``) inserts each test
file's directory at ``sys.path[0]``, ahead of this package.

Nothing here touches the GPU; the script's own imports do, after the paths
are set.
"""
from __future__ import annotations

import os
import runpy
import sys

PKG = os.path.dirname(os.path.abspath(__file__))

USAGE = ("usage: run_reference.py SCRIPT [args...]\n"
         "       run_reference.py -m MODULE [args...]")


def search_path(first_dir: str, rest: list) -> list:
    """sys.path for the harness: this package, then `first_dir`, then the
    rest in order, without repeats and without the launcher's own entries
    for the current directory ('' and '.')."""
    out = []
    for p in [PKG, first_dir] + list(rest):
        if p in ("", "."):
            continue
        p = os.path.abspath(p)
        if p not in out:
            out.append(p)
    return out


def main(argv: list) -> int:
    if not argv or argv[0] in ("-h", "--help"):
        print(USAGE)
        return 0 if argv else 2
    # sys.path[0] is this file's directory (python put it there); drop it and
    # rebuild the order explicitly.
    rest = sys.path[1:]
    if argv[0] == "-m":
        if len(argv) < 2:
            print(USAGE, file=sys.stderr)
            return 2
        module, args = argv[1], argv[2:]
        if module == "pytest" and not any(a.startswith("--import-mode") for a in args):
            args = ["--import-mode=append"] + args
        sys.path[:] = search_path(os.getcwd(), rest)
        sys.argv = [module] + args
        try:
            runpy.run_module(module, run_name="__main__", alter_sys=True)
        except SystemExit as e:  # pytest and argparse-style scripts exit through here
            return _code(e)
        return 0
    script, args = argv[0], argv[1:]
    if not os.path.isfile(script):
        print(f"run_reference.py: no such script: {script}", file=sys.stderr)
        return 2
    sys.path[:] = search_path(os.path.dirname(os.path.abspath(script)), rest)
    sys.argv = [script] + args
    try:
        runpy.run_path(script, run_name="__main__")
    except SystemExit as e:
        return _code(e)
    return 0


def _code(e: SystemExit) -> int:
    if e.code is None:
        return 0
    if isinstance(e.code, int):
        return e.code
    print(e.code, file=sys.stderr)
    return 1


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
