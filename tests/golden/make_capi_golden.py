"""Records the golden output of verbo_generate on the reference's tiny test models, from the
reference's own sampler (the unswapped build of tests/swap/build_swap.py), and copies those models
into tests/golden/tiny/ as fixtures (they are data files the reference's own tests hold,
tests/data/tiny-llama and tests/data/tiny-qwen2), so that a machine without the reference tree can
run the same scenarios through the swapped build.

    python tests/golden/make_capi_golden.py

Writes tests/golden/capi_generate_golden.jsonl (one line per scenario of
tests/swap/capi_generate.cpp) and tests/golden/tiny/<model>/*.
"""
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "tests" / "swap"))
import build_swap  # noqa: E402

MODELS = ("tiny-llama", "tiny-qwen2")


def copy_models():
    for m in MODELS:
        dst = HERE / "tiny" / m
        dst.mkdir(parents=True, exist_ok=True)
        for f in sorted((build_swap.REF / "tests" / "data" / m).iterdir()):
            shutil.copyfile(f, dst / f.name)


def main():
    copy_models()
    ref = build_swap.OUT / "ref" / "capi_generate"
    if not ref.is_file():
        build_swap.build_kind("ref")
    out = subprocess.run([str(ref), str(HERE / "tiny")], check=True, capture_output=True, text=True).stdout
    (HERE / "capi_generate_golden.jsonl").write_text(out)
    print(out)


if __name__ == "__main__":
    main()
