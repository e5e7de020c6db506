"""Records the CLI golden: verbo's own command line (`verbo run`, reference cli/main.cpp:39-66, which
calls generate at :58) built unswapped from the reference's sources (tests/swap/build_swap.py:
tests/swap/_build/ref/verbo), run on the reference's tiny test models over scenarios covering the
sampler's paths (greedy, top-k, top-k off with top-p, min-p, penalties; raw text and the chat
template). tests/test_swap_gpu.py runs the same commands on the build with the GPU sampler swapped in
and compares its output byte for byte.

    python tests/swap/build_swap.py && python tests/golden/make_cli_golden.py

Writes tests/golden/cli_run_golden.jsonl: per scenario its arguments and the base64 of stdout.
"""
import base64
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "cli_run_golden.jsonl"

# (name, model, arguments after `verbo run -m MODEL`); one thread, so that the CPU model is the same
# computation on any host
SCENARIOS = [
    ("greedy_raw", "tiny-llama", ["--raw", "-p", "The quick brown fox", "-n", "24", "--temp", "0"]),
    ("greedy_chat", "tiny-qwen2", ["-p", "hello there", "-n", "24", "--temp", "0"]),
    ("topk_seeded", "tiny-llama", ["--raw", "-p", "Once upon a time", "-n", "32", "--temp", "0.8", "--top-k", "40",
                                   "--seed", "7"]),
    ("topp_only", "tiny-qwen2", ["--raw", "-p", "A B C", "-n", "32", "--temp", "1.0", "--top-k", "0", "--top-p", "0.9",
                                 "--seed", "3"]),
    ("minp_penalty", "tiny-qwen2", ["-p", "count to ten", "-n", "32", "--temp", "0.7", "--min-p", "0.05", "--repeat",
                                    "1.3", "--seed", "11"]),
    ("f32_sampled", "tiny-llama", ["--raw", "-p", "x", "-n", "20", "-q", "f32", "--temp", "1.2", "--top-k", "300",
                                   "--top-p", "0.95", "--repeat", "1.1", "--seed", "99"]),
]


def command(exe, model, args):
    return [str(exe), "run", "-m", str(ROOT / "tests" / "golden" / "tiny" / model), "-t", "1", "--quiet", *args]


def main():
    exe = ROOT / "tests" / "swap" / "_build" / "ref" / "verbo"
    if not exe.is_file():
        sys.exit(f"{exe} is built by tests/swap/build_swap.py")
    with open(OUT, "w") as f:
        for name, model, args in SCENARIOS:
            out = subprocess.run(command(exe, model, args), check=True, capture_output=True, timeout=300).stdout
            f.write(json.dumps({"name": name, "model": model, "args": args,
                                "stdout_b64": base64.b64encode(out).decode()}) + "\n")
            print(name, len(out), "bytes")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
