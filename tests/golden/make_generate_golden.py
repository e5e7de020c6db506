"""Writes tests/golden/generate_golden.jsonl: the decode sequences of the reference's own
verbo::generate and verbo::Sampler (src/sampler.cpp, compiled from the reference tree by
oracle/Makefile into oracle/_ref/gen_ref) over the test double tests/generate/fake_verbo.cpp.

    make -C oracle ref && python tests/golden/make_generate_golden.py

One JSON line per scenario: tokens, Stats (prompt, gen, stopped), the session position and every
text chunk handed to the callback.
"""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]


def main():
    exe = ROOT / "oracle" / "_ref" / "gen_ref"
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    (ROOT / "tests" / "golden" / "generate_golden.jsonl").write_text(out)
    print(f"{len(out.splitlines())} scenarios")


if __name__ == "__main__":
    main()
