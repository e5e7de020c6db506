"""The reference-side swap, on the CPU: the two CMake blocks, taken from the integration notes
themselves, applied to a scratch copy of the reference tree, build every target
(`verbo`, `libverbo.so`, the `verbo` CLI, `verbo_tests`); `libverbo.so` then needs `libvsmp.so`,
leaves only those `verbo::Sampler` symbols undefined that `libvsmp.so` exports, and loads. The
unswapped build reproduces the committed verbo_generate golden. Skipped without the reference
tree."""
import ctypes
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "swap"))
import build_swap  # noqa: E402

pytestmark = pytest.mark.skipif(not build_swap.REF.is_dir(), reason="reference tree absent")


def _symbols(lib, undefined):
    flag = "--undefined-only" if undefined else "--defined-only"
    out = subprocess.run(["nm", "-D", "-C", flag, str(lib)], check=True, capture_output=True, text=True).stdout
    # "                 U name" or "0000000000094530 T name"
    return {line.strip()[2:] if undefined else line.split(" ", 2)[-1] for line in out.splitlines() if line.strip()}


def test_cmake_blocks_patch_the_reference():
    before, after = build_swap.cmake_blocks()
    text = (build_swap.REF / "CMakeLists.txt").read_text()
    patched = build_swap.patch_cmakelists(text, before, after)
    assert patched.index("VERBO_GPU_SAMPLER") < patched.index("add_library(verbo_obj OBJECT")
    assert patched.rindex("target_link_libraries(verbo PUBLIC ${VSMP_LIB})") > patched.index("add_library(verbo_shared")
    assert "verbo_amd/../include" not in patched and "VSMP_DIR}/include" not in patched


def test_swapped_reference_builds_and_links(tmp_path):
    src, out = tmp_path / "verbo", tmp_path / "build"
    build_swap.scratch_tree(src, swap=True)
    with open(tmp_path / "build.log", "w") as log:
        build_swap.cmake_build(src, out, swap=True, log=log)
    for t in ("libverbo.a", "libverbo.so", "verbo", "verbo_tests"):
        assert (out / t).is_file(), t
    lib = out / "libverbo.so"
    dyn = subprocess.run(["readelf", "-d", str(lib)], check=True, capture_output=True, text=True).stdout
    assert "[libvsmp.so]" in dyn
    undef = {s for s in _symbols(lib, True) if s.startswith("verbo::")}
    assert "verbo::Sampler::pick(float const*, int)" in undef
    assert all(s.startswith("verbo::Sampler::") for s in undef), undef
    exported = _symbols(ROOT / "verbo_amd" / "libvsmp.so", False)
    assert undef <= exported, undef - exported
    for exe in ("verbo", "verbo_tests"):
        ldd = subprocess.run(["ldd", str(out / exe)], check=True, capture_output=True, text=True).stdout
        assert "libvsmp.so =>" in ldd and "not found" not in ldd, ldd
    v = ctypes.CDLL(str(lib))
    v.verbo_version.restype = ctypes.c_char_p
    assert v.verbo_version() == b"0.1.0"


def test_unswapped_reference_reproduces_the_generate_golden(tmp_path):
    """The golden that the GPU test compares the swapped build with is what the reference's own
    sampler produces (tests/golden/make_capi_golden.py)."""
    drv = build_swap.OUT / "ref" / "capi_generate"
    if not drv.is_file():
        drv = build_swap.build_kind("ref", tmp_path / "ref") / "capi_generate"
    got = subprocess.run([str(drv), str(ROOT / "tests" / "golden" / "tiny")], check=True, capture_output=True,
                         text=True, timeout=120).stdout
    gold = (ROOT / "tests" / "golden" / "capi_generate_golden.jsonl").read_text()
    assert [json.loads(x) for x in got.splitlines()] == [json.loads(x) for x in gold.splitlines()]
