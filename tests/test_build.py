"""The library build fails loudly: a source that does not compile fails `make`,
and no older object of the same name survives to be linked."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flashmaxsim.jl_amd")
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None,
                                reason="needs hipcc and make")


def _make_object(tmp_path, name, source):
    src, obj = tmp_path / "src", tmp_path / "obj"
    src.mkdir(exist_ok=True)
    obj.mkdir(exist_ok=True)
    (src / f"{name}.hip").write_text(source)
    target = obj / f"{name}.o"
    r = subprocess.run(["make", "-B", "-C", PKG, f"SRC={src}", f"OBJ={obj}", str(target)],
                       capture_output=True, text=True, timeout=600)
    return r, target


def test_broken_source_fails_make_and_drops_the_stale_object(tmp_path):
    (tmp_path / "obj").mkdir()
    stale = tmp_path / "obj" / "broken.o"
    stale.write_text("an object from an earlier build")
    r, target = _make_object(tmp_path, "broken", "int broken( {\n")
    assert r.returncode != 0, r.stdout + r.stderr
    assert "error" in r.stderr
    assert not target.exists(), "a failed compile left an object behind"


def test_good_source_builds(tmp_path):
    r, target = _make_object(
        tmp_path, "good",
        "#include <hip/hip_runtime.h>\n"
        "__global__ void k(float* x) { x[threadIdx.x] = 1.0f; }\n")
    assert r.returncode == 0, r.stdout + r.stderr
    assert target.exists()
    assert "packed-fp32-ops' is not a recognized feature" not in r.stderr
