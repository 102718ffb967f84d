"""The HIP library's build fails when a source fails to compile.

A copy of the package's Makefile, csrc/ and include/ is built in a temporary
directory with every object already present (empty stand-ins, newer than
their sources), then one source gets a syntax error: make must return
non-zero, leave no object for that source and not relink the library.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import time
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "montlok.cpp_amd"


@pytest.mark.skipif(not Path("/opt/rocm/bin/hipcc").exists(), reason="hipcc not installed")
def test_make_fails_on_a_broken_source(tmp_path):
    pkg = tmp_path / "pkg"
    (pkg / "_build").mkdir(parents=True)
    shutil.copy(PKG / "Makefile", pkg / "Makefile")
    shutil.copytree(PKG / "csrc", pkg / "csrc")
    shutil.copytree(ROOT / "include", tmp_path / "include")
    lib = pkg / "montlok" / "rdt" / "lib" / "libmlk_hip.so"
    lib.parent.mkdir(parents=True)
    past = time.time() - 3600
    for src in list((pkg / "csrc").iterdir()) + list((tmp_path / "include").iterdir()):
        os.utime(src, (past, past))
    for src in (pkg / "csrc").glob("*.hip"):
        (pkg / "_build" / f"{src.stem}.o").write_bytes(b"stale object")
    lib.write_bytes(b"stale library")
    # Only status.o is older than its source now; its compile must fail the build.
    with open(pkg / "csrc" / "status.hip", "a") as f:
        f.write("\nthis is not C++ ;\n")
    out = subprocess.run(["make", "-C", str(pkg)], capture_output=True, text=True, timeout=300)
    assert out.returncode != 0, out.stdout + out.stderr
    assert "hipcc failed" in out.stderr
    assert not (pkg / "_build" / "status.o").exists()
    assert lib.read_bytes() == b"stale library"


def test_build_entry_raises_on_make_failure(monkeypatch):
    import __graft_entry__ as ge

    def fake_run(*a, **k):
        return subprocess.CompletedProcess(a, 2, "", "hipcc failed (1)")

    monkeypatch.setattr(ge.subprocess, "run", fake_run)
    with pytest.raises(RuntimeError, match="failed"):
        ge._make("-C", str(PKG))
