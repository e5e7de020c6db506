"""Builds verbo (the reference) with the MI355X sampler swapped in by the two CMake blocks that the
repository's integration notes give a maintainer (read from that file, so that the notes are what is
built).

    python tests/swap/build_swap.py            # both builds and the drivers
    python tests/swap/build_swap.py swap       # the swapped build only

- swap: a scratch copy of the reference tree (in a temporary directory outside this repository)
  with the two CMake blocks applied, configured with -DVERBO_GPU_SAMPLER=ON and
  -DVSMP_DIR=<this checkout>, built into tests/swap/_build/swap: libverbo.so, libverbo.a, the
  `verbo` CLI and `verbo_tests` (the reference's own test binary).
- ref: the same tree without the blocks, built into tests/swap/_build/ref; its libverbo.so records
  the golden output of the verbo_generate driver.
- driver: tests/swap/capi_generate.cpp linked against each build's libverbo.so
  (tests/swap/_build/<kind>/capi_generate).

Both builds use -DVERBO_NATIVE=OFF, so that the binaries run on another x86-64 host and the CPU
forward pass of the tiny test models is the same machine code in both. Test infrastructure: run by
__graft_entry__.build() where the reference tree is present; nothing here is part of libvsmp.
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
REF = Path(os.environ.get("VSMP_REF_TREE", "/root/reference"))
OUT = HERE / "_build"
TARGETS = ["verbo", "verbo_shared", "verbo_cli", "verbo_tests"]


def cmake_blocks(integration=ROOT / "INTEGRATION.md"):
    """The two ```cmake blocks of the integration notes (before add_library(verbo_obj), after the
    targets), identified by their first comment line."""
    blocks = re.findall(r"```cmake\n(.*?)```", integration.read_text(), re.S)
    before = [b for b in blocks if b.startswith("# vsmp: before add_library(verbo_obj")]
    after = [b for b in blocks if b.startswith("# vsmp: after the targets")]
    if len(before) != 1 or len(after) != 1:
        raise RuntimeError(f"{integration} must hold exactly one 'before' and one 'after' cmake block")
    return before[0], after[0]


def patch_cmakelists(text, before, after):
    """The reference's CMakeLists.txt with `before` inserted right before add_library(verbo_obj ...)
    and `after` appended at the end."""
    at = text.index("add_library(verbo_obj OBJECT")
    return text[:at] + before + "\n" + text[at:] + "\n" + after


def scratch_tree(dst, swap):
    """A copy of the reference tree at dst (read-only files made writable), patched when `swap`."""
    shutil.copytree(REF, dst, symlinks=True, ignore=shutil.ignore_patterns(".git", "build*"))
    for p in Path(dst).rglob("*"):
        if not p.is_symlink():
            p.chmod(p.stat().st_mode | 0o200)
    Path(dst).chmod(0o755)
    if swap:
        cm = Path(dst) / "CMakeLists.txt"
        cm.write_text(patch_cmakelists(cm.read_text(), *cmake_blocks()))


def cmake_build(src, out, swap, jobs=None, log=None):
    """Configure and build TARGETS of the tree at src into out."""
    jobs = jobs or min(8, os.cpu_count() or 1)
    cfg = ["cmake", "-S", str(src), "-B", str(out), "-DCMAKE_BUILD_TYPE=Release", "-DVERBO_NATIVE=OFF",
           "-DVERBO_TESTS=ON"]
    if swap:
        cfg += ["-DVERBO_GPU_SAMPLER=ON", f"-DVSMP_DIR={ROOT}"]
    kw = dict(check=True, stdout=log or subprocess.DEVNULL, stderr=subprocess.STDOUT if log else None)
    subprocess.run(cfg, **kw)
    subprocess.run(["cmake", "--build", str(out), "-j", str(jobs), "--target", *TARGETS], **kw)


def build_kind(kind, out=None):
    """The swapped ('swap') or unswapped ('ref') build into out (default tests/swap/_build/<kind>)."""
    out = Path(out or OUT / kind)
    if out.exists():
        shutil.rmtree(out)
    with tempfile.TemporaryDirectory(prefix=f"verbo-{kind}-") as tmp:
        src = Path(tmp) / "verbo"
        scratch_tree(src, swap=kind == "swap")
        cmake_build(src, out, swap=kind == "swap")
    build_driver(out)
    return out


def build_driver(build):
    """tests/swap/capi_generate.cpp against the C ABI header of the reference and build/libverbo.so."""
    exe = Path(build) / "capi_generate"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-I", str(REF / "include"), "-o", str(exe),
                    str(HERE / "capi_generate.cpp"), "-L", str(build), "-lverbo", f"-Wl,-rpath,{Path(build).resolve()}"],
                   check=True)
    return exe


def main(argv):
    kinds = argv[1:] or ["swap", "ref"]
    if not REF.is_dir():
        print(f"{REF} is absent: nothing to build", file=sys.stderr)
        return 0
    for k in kinds:
        print(build_kind(k), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
