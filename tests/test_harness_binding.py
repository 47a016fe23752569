"""The reference's own harness must bind to this build unchanged.

Its scripts import ``submission`` (the entry points), ``workloads`` (their
shape tables) and ``reference.reference`` (the oracle) by bare module name
(track-01/test_correctness.py:12-14, track-01/bench.py:11-13,
track-01/profile.py:9-10, track-02/test_correctness.py:12-14,
track-03/test_correctness.py:9-11), and are run as ``python <script>`` from
inside the track, or under pytest (track-03). Both put the track's directory
ahead of ``PYTHONPATH``, so the documented commands go through
``kernelgen-challenge_amd/run_reference.py``, which puts the package first.

The tests run those commands for real, in CPU subprocesses, on a stand-in
track directory: a ``submission.py`` standing for the track's Triton file, a
``workloads.py``, a ``reference/`` package, and harness scripts that report
where each import resolved. Nothing of the reference is imported or run; the
reference's own scripts are only parsed as text (skipped where the reference
is not mounted), to check that every name they take from ``submission``
exists here.
"""
import ast
import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "kernelgen-challenge_amd")
LAUNCHER = os.path.join(PKG, "run_reference.py")
REFERENCE = "/root/reference"

# every top-level module the reference's harness scripts import
HARNESS_IMPORTS = {"submission", "reference", "workloads", "torch", "triton", "pytest",
                   "sys", "math", "argparse"}
HARNESS_SCRIPTS = ["track-01/test_correctness.py", "track-01/bench.py", "track-01/profile.py",
                   "track-02/test_correctness.py", "track-02/bench.py", "track-02/profile.py",
                   "track-03/test_correctness.py", "track-03/test_reference.py",
                   "track-03/test_workloads.py"]

# The stand-in harness script: the same three imports as the reference's
# (track-01/test_correctness.py:12-14), then a report of where they resolved.
SCRIPT = '''
import json, sys
from reference.reference import sparse_attn as ref_attn
from submission import sparse_attn as our_attn
from workloads import WHERE
import reference.reference, submission, workloads
print("RESOLVED " + json.dumps({"submission": submission.__file__,
                                "workloads": workloads.__file__,
                                "reference": reference.reference.__file__,
                                "argv": sys.argv[1:], "name": __name__}))
'''

# The stand-in pytest harness (track-03/test_correctness.py:9-11 imports the
# same way at module level).
PYTEST_MODULE = '''
import json, os
from submission import fused_moe as fused_moe_sub
from reference.reference import sparse_attn as ref
from workloads import WHERE
import submission, workloads, reference.reference

def test_where_imports_resolved():
    with open(os.environ["BINDING_REPORT"], "w") as f:
        json.dump({"submission": submission.__file__, "workloads": workloads.__file__,
                   "reference": reference.reference.__file__}, f)
'''


@pytest.fixture()
def track(tmp_path):
    """A stand-in track directory."""
    t = tmp_path / "track-01"
    (t / "reference").mkdir(parents=True)
    (t / "submission.py").write_text("raise ImportError('the track\\'s own submission was imported')\n")
    (t / "workloads.py").write_text("WHERE = __file__\n")
    (t / "reference" / "__init__.py").write_text("")
    (t / "reference" / "reference.py").write_text("def sparse_attn(*a):\n    pass\n")
    (t / "test_correctness.py").write_text(SCRIPT)
    (t / "test_binding.py").write_text(PYTEST_MODULE)
    return t


def _env(**extra):
    env = dict(os.environ)
    env.pop("PYTHONPATH", None)
    env.update(extra)
    return env


def _resolved(out):
    line = [ln for ln in out.splitlines() if ln.startswith("RESOLVED ")]
    assert line, out
    return json.loads(line[-1][len("RESOLVED "):])


def _assert_bound(where, track):
    assert os.path.dirname(where["submission"]) == PKG, where
    assert os.path.dirname(where["workloads"]) == str(track), where
    assert os.path.dirname(os.path.dirname(where["reference"])) == str(track), where


def test_plain_python_binds_the_track_not_the_package(track):
    """Why the launcher exists: ``PYTHONPATH=<pkg> python script.py`` puts the
    script's directory first, so the track's own submission.py wins."""
    r = subprocess.run([sys.executable, "test_correctness.py"], cwd=track, text=True,
                       capture_output=True, env=_env(PYTHONPATH=PKG), timeout=300)
    assert r.returncode != 0 and "the track's own submission was imported" in r.stderr


def test_launcher_binds_a_script(track):
    """``python <pkg>/run_reference.py test_correctness.py [args]`` run in the
    track: submission from the package, workloads and reference from the track,
    the script runs as __main__ with its own arguments."""
    r = subprocess.run([sys.executable, LAUNCHER, "test_correctness.py", "--x", "1"], cwd=track,
                       text=True, capture_output=True, env=_env(), timeout=300)
    assert r.returncode == 0, r.stderr
    where = _resolved(r.stdout)
    _assert_bound(where, track)
    assert where["argv"] == ["--x", "1"] and where["name"] == "__main__"


def test_launcher_binds_a_script_from_elsewhere(track, tmp_path):
    """The script's directory, not the current one, is the second entry."""
    r = subprocess.run([sys.executable, LAUNCHER, str(track / "test_correctness.py")],
                       cwd=tmp_path, text=True, capture_output=True, env=_env(), timeout=300)
    assert r.returncode == 0, r.stderr
    _assert_bound(_resolved(r.stdout), track)


def test_launcher_binds_pytest(track, tmp_path):
    """``python <pkg>/run_reference.py -m pytest test_x.py`` in the track."""
    report = tmp_path / "report.json"
    r = subprocess.run([sys.executable, LAUNCHER, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        "test_binding.py"], cwd=track, text=True, capture_output=True,
                       env=_env(BINDING_REPORT=str(report)), timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    _assert_bound(json.loads(report.read_text()), track)


def test_pytest_console_script_with_append_mode_binds(track, tmp_path):
    """The documented alternative for the pytest harness:
    ``PYTHONPATH=<pkg> pytest --import-mode=append test_x.py``."""
    pytest_bin = os.path.join(os.path.dirname(sys.executable), "pytest")
    if not os.path.exists(pytest_bin):
        import shutil
        pytest_bin = shutil.which("pytest")
    if not pytest_bin:
        pytest.skip("no pytest console script")
    report = tmp_path / "report.json"
    r = subprocess.run([pytest_bin, "-q", "-p", "no:cacheprovider", "--import-mode=append",
                        "test_binding.py"], cwd=track, text=True, capture_output=True,
                       env=_env(PYTHONPATH=PKG, BINDING_REPORT=str(report)), timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    _assert_bound(json.loads(report.read_text()), track)


def test_launcher_usage_errors():
    r = subprocess.run([sys.executable, LAUNCHER], text=True, capture_output=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stdout
    r = subprocess.run([sys.executable, LAUNCHER, "no_such_script.py"], text=True,
                       capture_output=True, timeout=60)
    assert r.returncode == 2 and "no such script" in r.stderr


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
def test_reference_harness_names_exist(script):
    """Every import of the reference's harness scripts is one of the modules
    the launcher arranges, and every name they take from ``submission``
    exists in this package's ``submission``."""
    path = os.path.join(REFERENCE, script)
    if not os.path.exists(path):
        pytest.skip(f"{script} not in this reference")
    import submission
    for module, names in _imports_of(path):
        top = module.split(".")[0]
        assert top in HARNESS_IMPORTS, f"{script} imports {module}: extend HARNESS_IMPORTS"
        if top == "submission":
            for n in names:
                assert hasattr(submission, n), f"{script}: submission.{n} missing"
