"""The drop-in claim, kept true by a test: the HIP backend sources compile against the reference's
own headers (include/vknn/*.h of katolikov/vknn) once the five additive lines a maintainer makes
are applied, and fail without them for exactly those names.

The reference headers are copied into a temporary directory (never into the repository), patched
there, and `g++ -fsyntax-only` runs hip_backend.cpp and tune_cache.cpp against them with the
reference's own src/ on the include path. Skipped where the reference tree is absent (the GPU box).
"""
import os
import re
import shutil
import subprocess

import pytest

REF = "/root/reference"
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "vknn_amd", "csrc", "host")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "include", "vknn")) or shutil.which("g++") is None,
                                reason="reference headers or g++ not available")

# (header, regex anchor, replacement): the five additions of the integration guide
ADDITIONS = [
    ("backend_kind.h", r"enum class BackendKind \{ Vulkan = 0, Cpu = 1 \};", "enum class BackendKind { Vulkan = 0, Cpu = 1, Hip = 2 };"),
    ("op_record.h", r"(bool\s+fellBack\s*=\s*false;[^\n]*\n)", r"\1        double flops = 0.0;\n"),
    ("config_struct.h", r"(struct Config \{\n)", r"\1        bool hipGraphs = true;\n        int profileReps = 1;\n        bool hipBranches = true;\n"),
]


def _tree(tmp, patched):
    inc = tmp / ("patched" if patched else "plain")
    shutil.copytree(os.path.join(REF, "include"), inc)
    if patched:
        for name, pat, rep in ADDITIONS:
            p = inc / "vknn" / name
            text = p.read_text()
            new, n = re.subn(pat, rep, text, count=1)
            assert n == 1, f"anchor for the {name} addition not found: the reference header changed"
            p.write_text(new)
    # vkhip.h alone from this repository (its own vknn/ headers must not shadow the reference's)
    abi = tmp / "abi"
    abi.mkdir(exist_ok=True)
    shutil.copy(os.path.join(ROOT, "include", "vkhip.h"), abi / "vkhip.h")
    return inc, abi


def _compile(inc, abi, src):
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-I", str(inc), "-I", os.path.join(REF, "src"), "-I", HOST, "-I", str(abi),
           os.path.join(HOST, src)]
    return subprocess.run(cmd, capture_output=True, text=True, env=dict(os.environ, LC_ALL="C", LANG="C"))


@pytest.mark.parametrize("src", ["hip_backend.cpp", "tune_cache.cpp"])
def test_backend_compiles_against_patched_reference_headers(tmp_path, src):
    inc, abi = _tree(tmp_path, patched=True)
    r = _compile(inc, abi, src)
    assert r.returncode == 0, r.stderr[-4000:]


def test_unpatched_reference_headers_fail_only_on_the_five_additions(tmp_path):
    """Without the additions, the only errors name the added identifiers."""
    inc, abi = _tree(tmp_path, patched=False)
    r = _compile(inc, abi, "hip_backend.cpp")
    assert r.returncode != 0
    errors = [ln for ln in r.stderr.splitlines() if ": error:" in ln]
    assert errors, r.stderr[-2000:]
    allowed = ("Hip", "hipGraphs", "profileReps", "hipBranches", "flops")
    for ln in errors:
        assert any(f"'{a}'" in ln for a in allowed), ln
    named = {a for a in allowed if any(f"'{a}'" in ln for ln in errors)}
    assert named == set(allowed), named
