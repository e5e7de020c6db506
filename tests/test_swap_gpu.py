"""verbo with the MI355X sampler swapped in (the integration notes' CMake blocks; built by
tests/swap/build_swap.py into tests/swap/_build/swap), run on the GPU:

- verbo_generate (reference src/capi.cpp:131-151) through the swapped libverbo.so on the
  reference's tiny test models equals what the reference's own sampler produced
  (tests/golden/capi_generate_golden.jsonl): greedy and sampled scenarios, penalties, min-p, top-p,
  a callback that stops;
- the reference's own test binary (tests/test_core.cpp) linked against the swap passes every
  group; its sampler (:454-496), generate (:498-536) and C-ABI (:543-589) groups then call the GPU
  sampler. The tiny models are the reference's test data, committed as fixtures.
"""
import json
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SWAP = ROOT / "tests" / "swap" / "_build" / "swap"
TINY = ROOT / "tests" / "golden" / "tiny"

pytestmark = pytest.mark.gpu


def _need(p):
    assert p.is_file(), f"{p} is built by tests/swap/build_swap.py (run by __graft_entry__.build())"


def test_verbo_generate_through_the_swapped_build():
    drv = SWAP / "capi_generate"
    _need(drv)
    print("swapped verbo_generate", flush=True)
    got = subprocess.run([str(drv), str(TINY)], check=True, capture_output=True, text=True, timeout=120).stdout
    gold = [json.loads(x) for x in (ROOT / "tests" / "golden" / "capi_generate_golden.jsonl").read_text().splitlines()]
    got = [json.loads(x) for x in got.splitlines()]
    assert [g["name"] for g in got] == [g["name"] for g in gold]
    bad = [(a["name"], a, b) for a, b in zip(got, gold) if a != b]
    assert not bad, bad[:2]


def test_reference_test_binary_on_the_gpu_sampler(tmp_path):
    exe = SWAP / "verbo_tests"
    _need(exe)
    (tmp_path / "tests").mkdir()
    (tmp_path / "tests" / "data").symlink_to(TINY)
    print("swapped verbo_tests", flush=True)
    r = subprocess.run([str(exe)], cwd=tmp_path, capture_output=True, text=True, timeout=240)
    out = r.stdout
    assert r.returncode == 0 and "0 failure(s)" in out, out[-2000:] + r.stderr[-2000:]
    lines = [x.strip() for x in out.splitlines()]
    for group in ("sampler", "generate", "capi"):
        assert lines[lines.index(group) + 1] == "ok", group


def test_verbo_cli_run_through_the_swapped_build():
    """verbo's own command line (`verbo run`, reference cli/main.cpp:39-66, generate at :58) linked
    against the GPU sampler prints what the unswapped build printed (tests/golden/cli_run_golden.jsonl,
    recorded by tests/golden/make_cli_golden.py), byte for byte: greedy, top-k, top-p only, min-p with
    penalties, raw text and the chat template, q8 and f32 models."""
    import base64
    import sys

    sys.path.insert(0, str(ROOT / "tests" / "golden"))
    from make_cli_golden import command

    exe = SWAP / "verbo"
    _need(exe)
    gold = [json.loads(x) for x in (ROOT / "tests" / "golden" / "cli_run_golden.jsonl").read_text().splitlines()]
    assert len(gold) >= 6
    for g in gold:
        print("swapped verbo run:", g["name"], flush=True)
        out = subprocess.run(command(exe, g["model"], g["args"]), check=True, capture_output=True, timeout=120).stdout
        assert out == base64.b64decode(g["stdout_b64"]), (g["name"], out)
