"""Batched decoding (verbo_amd.decode.BatchDecoder over vsmp_bsampler): 24 sequences with their own
options, prompts and repeat_last windows decoded together on the GPU, every history appended on the
device, against 24 independent reference Samplers decoding the same sequences
(tests/golden/decode_golden.jsonl, recorded from the compiled reference by
tests/golden/make_decode_golden.py). The CPU test pins that golden with the oracle."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from verbo_amd.workloads import DecodeCase

GOLD = Path(__file__).resolve().parent / "golden" / "decode_golden.jsonl"


def _gold():
    return [json.loads(x) for x in GOLD.read_text().splitlines()]


def test_oracle_reproduces_the_decode_golden():
    """The same decode with the oracle's Sampler pieces (seeding, xorshift draws, accept trimming,
    pick) in place of the reference's."""
    c = DecodeCase()
    st, hist, cfg = [], [], []
    for r in range(c.n):
        o = c.opts[r]
        cfg.append(O.sampling(temp=o["temp"], top_k=o["top_k"], top_p=o["top_p"], min_p=o["min_p"], repeat=o["repeat"],
                              repeat_last=c.repeat_last[r], seed=o["seed"]))
        st.append(O.rng_seed(o["seed"]))
        h = np.zeros(4 * c.repeat_last[r] + 64 + len(c.prompts[r]), np.int32)
        n = 0
        lib = O.load_oracle()
        for t in c.prompts[r]:
            n = lib.vo_accept(h.ctypes.data_as(O._P), n, int(t), c.repeat_last[r])
        hist.append([h, n])
    toks = [[] for _ in range(c.n)]
    stopped = [False] * c.n
    live = [c.opts[r]["max_tokens"] > 0 for r in range(c.n)]
    last = np.full(c.n, -1)
    step = 0
    while any(live):
        lg = c.logits(step, last)
        for r in range(c.n):
            if not live[r]:
                continue
            u = O.rng_unit(st[r]) if cfg[r].temp > 0 else 0.0
            h, n = hist[r]
            t = O.pick(lg[r], cfg[r], h[:n], u)[0]
            if t in c.stop_ids:
                live[r], stopped[r] = False, True
                continue
            hist[r][1] = lib.vo_accept(h.ctypes.data_as(O._P), n, int(t), c.repeat_last[r])
            toks[r].append(t)
            last[r] = t
            if len(toks[r]) >= c.opts[r]["max_tokens"]:
                live[r] = False
        step += 1
    assert [{"row": r, "toks": toks[r], "stopped": stopped[r]} for r in range(c.n)] == _gold()


@pytest.mark.gpu
def test_batched_decode_equals_independent_reference_samplers():
    import torch

    from verbo_amd.decode import BatchDecoder, Opts

    c = DecodeCase()
    dec = BatchDecoder([Opts(**o) for o in c.opts], c.V, repeat_last=c.repeat_last)

    def logits_fn(step, last, live):
        return torch.from_numpy(c.logits(step, last)).cuda()

    print("batched decode", c.n, "sequences", flush=True)
    res = dec.generate(c.prompts, logits_fn, stop_ids=c.stop_ids)
    got = [{"row": r, "toks": t, "stopped": s} for r, (t, s) in enumerate(res)]
    gold = _gold()
    bad = [(g["row"], g, w) for g, w in zip(got, gold) if g != w]
    assert not bad, bad[:2]
