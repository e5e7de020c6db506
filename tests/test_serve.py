"""Continuous batching (verbo_amd.decode.BatchDecoder.serve over vsmp_bsampler_admit / pick_rows /
accept_rows): 40 requests with their own options, prompts and repeat_last windows arrive over 60
steps (a third of them at once) at a decoder of 8 slots. Finished requests free their slots, queued
ones take them, and each step samples the live slots only. Every request's tokens equal those of its
own reference verbo::Sampler decoding it alone (tests/golden/serve_golden.jsonl, recorded from the
compiled reference by tests/golden/make_serve_golden.py); the CPU test pins that golden with the
oracle."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from verbo_amd.workloads import ServeCase

GOLD = Path(__file__).resolve().parent / "golden" / "serve_golden.jsonl"


def _gold():
    return [json.loads(x) for x in GOLD.read_text().splitlines()]


def test_oracle_reproduces_the_serve_golden():
    """Each request decoded alone with the oracle's Sampler pieces (seeding, xorshift draws, accept
    trimming, pick) in place of the reference's."""
    c = ServeCase()
    lib = O.load_oracle()
    got = []
    for j in range(c.n):
        o = c.opts[j]
        cfg = O.sampling(temp=o["temp"], top_k=o["top_k"], top_p=o["top_p"], min_p=o["min_p"], repeat=o["repeat"],
                         repeat_last=c.repeat_last[j], seed=o["seed"])
        st = O.rng_seed(o["seed"])
        h = np.zeros(4 * c.repeat_last[j] + 64 + len(c.prompts[j]), np.int32)
        n = 0
        for t in c.prompts[j]:
            n = lib.vo_accept(h.ctypes.data_as(O._P), n, int(t), c.repeat_last[j])
        toks, stopped, last, t = [], False, -1, 0
        while len(toks) < o["max_tokens"]:
            u = O.rng_unit(st) if cfg.temp > 0 else 0.0
            tok = O.pick(c.logits([j], [t], [last])[0], cfg, h[:n], u)[0]
            t += 1
            if tok in c.stop_ids:
                stopped = True
                break
            n = lib.vo_accept(h.ctypes.data_as(O._P), n, int(tok), c.repeat_last[j])
            toks.append(tok)
            last = tok
        got.append({"req": j, "toks": toks, "stopped": stopped})
    assert got == _gold()


def test_serve_case_shape():
    """The request stream needs more requests than slots, a burst larger than the slots, and
    requests that ask for nothing, so that queueing, slot reuse and the empty case all occur."""
    c = ServeCase()
    assert c.n > 2 * c.slots
    assert sum(a == 0 for a in c.arrival) > c.slots
    assert any(o["max_tokens"] == 0 for o in c.opts)
    assert all(o["seed"] != 0 for o in c.opts)  # seed 0 would stand for the clock


@pytest.mark.gpu
def test_continuous_batching_equals_requests_decoded_alone():
    import torch

    from helpers import log
    from verbo_amd.decode import BatchDecoder, Opts, Request

    c = ServeCase()
    reqs = [Request(c.prompts[j], Opts(**c.opts[j]), c.repeat_last[j], c.arrival[j]) for j in range(c.n)]
    dec = BatchDecoder.with_slots(c.slots, c.V)

    def logits_fn(js, steps, last):
        return torch.from_numpy(c.logits(js, steps, last)).cuda()

    log("serve", c.n, "requests over", c.slots, "slots")
    res = dec.serve(reqs, logits_fn, stop_ids=c.stop_ids)
    got = [{"req": j, "toks": t, "stopped": s} for j, (t, s) in enumerate(res)]
    gold = _gold()
    bad = [(g["req"], g, w) for g, w in zip(got, gold) if g != w]
    assert not bad, bad[:2]
    # the schedule: never more live slots than the decoder has, a slot held by one request at a time,
    # slots taken again after their requests finished, and only live requests sampled
    sched = dec.schedule
    assert max(len(s) for s in sched) == c.slots
    owner = {}
    users = {}
    for step in sched:
        slots = [s for _, s in step]
        assert len(set(slots)) == len(slots)
        for j, s in step:
            users.setdefault(s, []).append(j)
            owner.setdefault(j, s)
            assert owner[j] == s  # a request keeps its slot
    assert sum(len(set(u)) for u in users.values()) == sum(1 for o in c.opts if o["max_tokens"] > 0)
    assert max(len(set(u)) for u in users.values()) >= 3  # slots reused
    picks = sum(len(s) for s in sched)
    assert picks == sum(len(g["toks"]) + g["stopped"] for g in gold)  # one pick per generated or stop id
