"""The CMake build (CMakeLists.txt, cmake/Helix*.cmake): libhelix.a with the
code object embedded, and the C test that links it (tests/c/test_helix_c.c).

Counterpart of the reference's CMake build (CMakeLists.txt:37-114,
cmake/HelixEmbed.cmake:16-28, cmake/HelixEmbedRun.cmake:7-34). The builds here
embed the code object helix_amd/csrc/Makefile already compiled
(HELIX_CODE_OBJECT), so they take seconds; CMake's own hipcc --genco step is
the same compile the Makefile runs.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HSACO = os.path.join(ROOT, "helix_amd", "csrc", "_build", "helix_kernels.hsaco")

pytestmark = pytest.mark.skipif(not (shutil.which("cmake") and shutil.which("ninja")),
                                reason="cmake and ninja are needed")


@pytest.fixture(scope="module")
def cmake_build(tmp_path_factory):
    if not os.path.exists(HSACO):
        pytest.fail("helix_amd/csrc/_build/helix_kernels.hsaco is missing: run __graft_entry__.build()")
    b = tmp_path_factory.mktemp("cmake")
    for cmd in (["cmake", "-S", ROOT, "-B", str(b), "-G", "Ninja", f"-DHELIX_CODE_OBJECT={HSACO}"],
                ["cmake", "--build", str(b)]):
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return b


def test_static_library_embeds_code_object(cmake_build):
    lib = cmake_build / "libhelix.a"
    assert lib.exists()
    src = (cmake_build / "embed" / "helix_hsaco_data.c").read_text()
    body = src[src.index("{") + 1:src.index("};")]
    data = bytes(int(t, 16) for t in re.findall(r"0x([0-9a-f]{2})", body))
    assert data == open(HSACO, "rb").read()
    assert f"helix_hsaco_len = {len(data)};" in src
    names = subprocess.run(["nm", "-g", "--defined-only", str(lib)], capture_output=True, text=True).stdout
    for sym in ("helix_ctx_create", "helix_ctx_create_host", "helix_scan_encode", "helix_scan_encode_into",
                "helix_scan_encode_noalloc", "helix_scan_scratch_size", "helix_scan_supported",
                "helix_scan_desc_init", "helix_hsaco_data"):
        assert re.search(rf"\b[TDR] {sym}$", names, re.M), sym


def test_c_program_host_checks(cmake_build):
    r = subprocess.run([str(cmake_build / "test_helix_c"), "--host-only"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "host: config 0 scratch" in r.stdout and "test_helix_c: passed" in r.stdout


@pytest.mark.gpu
def test_c_program_encodes_on_gpu(cmake_build):
    """The C program's config-0 encodes on the fp32 and bf16 paths against the C oracle."""
    r = subprocess.run([str(cmake_build / "test_helix_c"), "--require-gpu"], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("gpu: ") == 2
