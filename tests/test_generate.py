"""verbo::generate (reference src/sampler.cpp:111-181) as a drop-in.

Both sides run the same deterministic test double (tests/generate/fake_verbo.cpp: Model, Session
and Detok behind verbo's interface) through a fixed list of decode scenarios: stop ids, stop
strings split across tokens (hold-back), a callback that stops, the context limit, max_tokens,
text held by the detokeniser and flushed, greedy and sampled picks with penalties.
- golden: the reference's own generate + Sampler, compiled from its sources (oracle/_ref/gen_ref),
  recorded in tests/golden/generate_golden.jsonl;
- ours: verbo_amd/csrc/generate.cpp + the GPU Sampler of libvsmp.so (tests/generate/gen_ours);
- ours, device-resident: vsmp::generate_device (verbo_amd/csrc/generate_device.cpp) over the same
  double with its logits copied to the device, as an LM head on the GPU would leave them; the draw
  stream and the history live on the device (tests/generate/gen_ours_device).
"""
import json
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden" / "generate_golden.jsonl"
GEN_REF = ROOT / "oracle" / "_ref" / "gen_ref"
GEN_OURS = ROOT / "tests" / "generate" / "gen_ours"
GEN_DEVICE = ROOT / "tests" / "generate" / "gen_ours_device"


def _lines(text):
    return [json.loads(x) for x in text.splitlines() if x.strip()]


def test_golden_is_the_compiled_reference():
    """The committed fixture is what the compiled reference prints (where it is built)."""
    gold = _lines(GOLDEN.read_text())
    assert len(gold) == 11
    if not GEN_REF.is_file():
        pytest.skip("oracle/_ref/gen_ref not built here")
    got = _lines(subprocess.run([str(GEN_REF)], check=True, capture_output=True, text=True, timeout=60).stdout)
    assert got == gold


def test_golden_invariants():
    """The fixture's sequences obey generate's contract: gen == len(toks) <= max_tokens, no
    text after a stop string, a callback-stopped run ends on the callback's refusal."""
    for g in _lines(GOLDEN.read_text()):
        assert g["gen"] == len(g["toks"])
        if g["name"] == "callback_stops":
            assert g["stopped"] and len(g["text"]) == 4
        if g["name"] == "ctx_limit":
            assert g["pos"] == 10 and not g["stopped"]
        if g["name"] == "stop_id":
            assert g["stopped"] and 3 not in g["toks"]
        if g["name"].startswith("stop_text"):
            assert g["stopped"]
            text = "".join(g["text"])
            assert "cd" not in text if g["name"] == "stop_text" else "abcd" not in text


@pytest.mark.gpu
def test_drop_in_generate_matches_reference():
    assert GEN_OURS.is_file(), "tests/generate/gen_ours is built by __graft_entry__.build()"
    got = _lines(subprocess.run([str(GEN_OURS)], check=True, capture_output=True, text=True, timeout=120).stdout)
    gold = _lines(GOLDEN.read_text())
    assert [g["name"] for g in got] == [g["name"] for g in gold]
    bad = [(a["name"], a, b) for a, b in zip(got, gold) if a != b]
    assert not bad, bad[:2]


@pytest.mark.gpu
def test_device_resident_generate_matches_reference():
    """Only the picked ids cross to the host: the sequences, Stats and text chunks still equal the
    reference's generate scenario by scenario."""
    assert GEN_DEVICE.is_file(), "tests/generate/gen_ours_device is built by __graft_entry__.build()"
    got = _lines(subprocess.run([str(GEN_DEVICE)], check=True, capture_output=True, text=True, timeout=120).stdout)
    gold = _lines(GOLDEN.read_text())
    assert [g["name"] for g in got] == [g["name"] for g in gold]
    bad = [(a["name"], a, b) for a, b in zip(got, gold) if a != b]
    assert not bad, bad[:2]
