"""The C-ABI library on the CPU: it loads, exports every symbol include/vsmp.h declares, and its
structs have the layouts the header and the reference fix. No GPU calls."""
import ctypes
import re
from pathlib import Path

import pytest

import verbo_amd as V

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    src = (ROOT / "include" / "vsmp.h").read_text()
    return re.findall(r"VSMP_API\s+[\w\s\*]+?\b(vsmp_\w+)\s*\(", src)


def test_library_exports_every_declared_symbol():
    lib = V.load_library()
    names = declared_symbols()
    assert len(names) == 32, names
    for n in names:
        assert hasattr(lib, n), n


def test_struct_layouts():
    # vsmp_params mirrors verbo::Sampling (reference include/verbo/verbo.hpp:56-64)
    assert ctypes.sizeof(V.Params) == 32
    assert [f for f, _ in V.Params._fields_] == ["temp", "top_k", "top_p", "min_p", "repeat", "repeat_last", "seed"]
    assert V.Params.seed.offset == 24
    assert ctypes.sizeof(V.RowInfo) == 72
    p = V.Params()
    assert (p.top_k, p.repeat_last, p.seed) == (40, 64, 0)
    assert abs(p.temp - 0.7) < 1e-7 and abs(p.top_p - 0.9) < 1e-7


def test_version_and_error_text():
    assert V.version() == V.__version__
    assert V.load_library().vsmp_last_error() == b""


def test_drop_in_header_keeps_sampler_layout():
    """The drop-in header declares Sampler's members in the reference's order (the reference
    compiles Sampler::cfg() inline into callers), and Sampling's fields and defaults."""
    h = (ROOT / "include" / "verbo" / "verbo.hpp").read_text()
    body = h[h.index("class Sampler {"):]
    body = body[:body.index("};")]
    members = re.findall(r"^\s+([\w:<>,\s\*]+?)\s+(\w+(?:\[2\])?);", body, re.M)
    assert [m[1] for m in members if not m[0].startswith("double")] == ["cfg_", "rng_[2]", "hist_", "buf_"]
    for line in ["float temp = 0.7f;", "int top_k = 40;", "float top_p = 0.9f;", "float min_p = 0.0f;",
                 "float repeat = 1.0f;", "int repeat_last = 64;", "std::uint64_t seed = 0;"]:
        assert line in h


@pytest.mark.skipif(not Path("/root/reference/include/verbo/verbo.hpp").is_file(), reason="reference tree absent")
def test_drop_in_types_have_the_reference_layout(tmp_path):
    """Every type the drop-in Sampler and generate share with verbo has the reference header's
    size and field offsets (tests/generate/layout.cpp built against both headers)."""
    import subprocess

    outs = []
    for inc in (ROOT / "include", Path("/root/reference/include")):
        exe = tmp_path / f"layout_{len(outs)}"
        subprocess.run(["g++", "-std=c++17", "-I", str(inc), "-o", str(exe), str(ROOT / "tests" / "generate" / "layout.cpp")],
                       check=True)
        outs.append(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    assert outs[0] == outs[1], outs
