"""The reference's own harness must bind to this build unchanged.

Its scripts import ``submission`` (the entry points), ``workloads`` (their
shape tables) and ``reference.reference`` (the oracle) by bare module name
(track-01/test_correctness.py:12-14, track-01/bench.py:11-13,
track-01/profile.py:9-10, track-02/test_correctness.py:12-14,
track-03/test_correctness.py:9-11). With ``kernelgen-challenge_amd/`` ahead
of the track's directory on ``sys.path``, ``submission`` must resolve here and
the other two to the track. So the package must not hold a module named like
any other import of those scripts, and ``submission`` must export every name
they take from it.

Module resolution is checked with ``importlib``'s path finder, which reads
directory listings only: nothing of the reference is imported or run. The
part that looks at the reference's scripts (as text) is skipped where the
reference is not mounted.
"""
import ast
import importlib.machinery
import os

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "kernelgen-challenge_amd")
REFERENCE = "/root/reference"

# every top-level module the reference's harness scripts import
HARNESS_IMPORTS = {"submission", "reference", "workloads", "torch", "triton", "pytest",
                   "sys", "math", "argparse"}
HARNESS_SCRIPTS = ["track-01/test_correctness.py", "track-01/bench.py", "track-01/profile.py",
                   "track-02/test_correctness.py", "track-02/bench.py", "track-02/profile.py",
                   "track-03/test_correctness.py", "track-03/test_reference.py",
                   "track-03/test_workloads.py"]


def package_modules():
    names = set()
    for f in os.listdir(PKG):
        path = os.path.join(PKG, f)
        if f.endswith(".py"):
            names.add(f[:-3])
        elif os.path.isdir(path) and os.path.exists(os.path.join(path, "__init__.py")):
            names.add(f)
    return names


def test_package_shadows_nothing_but_submission():
    clash = (package_modules() & HARNESS_IMPORTS) - {"submission"}
    assert not clash, f"package modules shadow the reference harness's imports: {clash}"
    assert "submission" in package_modules()


def test_submission_exports_every_track_entry_point():
    import submission
    for name in ("sparse_attn", "hc_split_sinkhorn", "fused_moe"):
        assert callable(getattr(submission, name, None)), name


def _imports_of(script):
    """(module, [names]) of every import statement of a harness script."""
    tree = ast.parse(open(script).read())
    out = []
    for node in ast.walk(tree):
        if isinstance(node, ast.ImportFrom) and node.module:
            out.append((node.module, [a.name for a in node.names]))
        elif isinstance(node, ast.Import):
            out.extend((a.name, []) for a in node.names)
    return out


@pytest.mark.skipif(not os.path.isdir(REFERENCE), reason="reference not mounted")
@pytest.mark.parametrize("script", HARNESS_SCRIPTS)
def test_reference_harness_resolves(script):
    path = os.path.join(REFERENCE, script)
    if not os.path.exists(path):
        pytest.skip(f"{script} not in this reference")
    track = os.path.dirname(path)
    search = [PKG, track]  # the documented order: the package first
    import submission
    for module, names in _imports_of(path):
        top = module.split(".")[0]
        assert top in HARNESS_IMPORTS, f"{script} imports {module}: extend HARNESS_IMPORTS"
        spec = importlib.machinery.PathFinder.find_spec(top, search)
        if top == "submission":
            assert spec is not None and os.path.dirname(spec.origin) == PKG
            for n in names:
                assert hasattr(submission, n), f"{script}: submission.{n} missing"
        elif top in ("workloads", "reference"):
            assert spec is not None, f"{script}: {top} not found"
            where = os.path.dirname(spec.origin)
            if top == "reference":  # a package: origin is its __init__.py
                where = os.path.dirname(where)
            assert where == track, f"{script}: {top} resolves to {where}, not the track"
        else:  # stdlib / third party: must not come from the package
            assert spec is None or not spec.origin or \
                os.path.dirname(spec.origin) != PKG, f"{script}: {top} shadowed"
