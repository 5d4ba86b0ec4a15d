"""The library build stops on a compile error (csrc/Makefile).

A source that does not compile must make ``make -B`` exit non-zero and leave
no object behind, so that ``__graft_entry__.build()`` (``make -B``,
``check=True``) can never link a stale object.  The check copies the Makefile,
one source and the headers into a scratch tree and breaks the source there.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "dwarf-v2_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def _scratch_tree(tmp_path):
    csrc = tmp_path / "pkg" / "csrc"
    csrc.mkdir(parents=True)
    for name in os.listdir(CSRC):
        if name.endswith((".h", "Makefile")):
            shutil.copy(os.path.join(CSRC, name), csrc / name)
    shutil.copytree(os.path.join(ROOT, "include"), tmp_path / "include")
    return csrc


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_compile_error_fails_make_and_removes_the_object(tmp_path):
    csrc = _scratch_tree(tmp_path)
    (csrc / "npci.hip").write_text('#include "common.h"\nthis line is not C++;\n')
    obj = csrc / "_build" / "npci.o"
    obj.parent.mkdir()
    obj.write_bytes(b"stale object from an earlier build")
    r = subprocess.run(["make", "-B", "-C", str(csrc), "_build/npci.o"], capture_output=True, text=True)
    assert r.returncode != 0, r.stdout + r.stderr
    assert "error" in (r.stdout + r.stderr)
    assert not obj.exists(), "a failed compile left the stale object in place"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_clean_source_builds_with_the_filtered_warning(tmp_path):
    csrc = _scratch_tree(tmp_path)
    (csrc / "npci.hip").write_text('#include "common.h"\nextern "C" int dwarf_build_probe(void) { return 7; }\n')
    r = subprocess.run(["make", "-B", "-C", str(csrc), "_build/npci.o"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert (csrc / "_build" / "npci.o").stat().st_size > 0
    # hipcc's output passes the filter onto make's stdout, beside the echoed recipe that names the filtered text
    warned = [ln for ln in (r.stdout + r.stderr).splitlines() if "recognized feature" in ln and "grep" not in ln]
    assert not warned, warned
