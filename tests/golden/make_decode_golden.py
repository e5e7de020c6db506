"""Records the multi-sequence decode golden: every sequence of verbo_amd.workloads.DecodeCase decoded
by its own reference verbo::Sampler (the reference's src/sampler.cpp compiled from its sources into
oracle/_ref/libvref.so), in verbo::generate's order (reference src/sampler.cpp:111-181: the prompt
accepted first; per step pick, a stop id ends the sequence unaccepted, any other id is accepted,
until max_tokens).

    make -C oracle ref && python tests/golden/make_decode_golden.py

Writes tests/golden/decode_golden.jsonl: per sequence its tokens and whether a stop id ended it.
"""
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT))

import oracle as O  # noqa: E402
from verbo_amd.workloads import DecodeCase  # noqa: E402

OUT = Path(__file__).resolve().parent / "decode_golden.jsonl"


def main():
    c = DecodeCase()
    smp = []
    for r in range(c.n):
        o = c.opts[r]
        s = O.RefSampler(O.sampling(temp=o["temp"], top_k=o["top_k"], top_p=o["top_p"], min_p=o["min_p"],
                                    repeat=o["repeat"], repeat_last=c.repeat_last[r], seed=o["seed"]))
        for t in c.prompts[r]:
            s.accept(int(t))
        smp.append(s)
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
            t = smp[r].pick(lg[r])
            if t in c.stop_ids:
                live[r], stopped[r] = False, True
                continue
            smp[r].accept(t)
            toks[r].append(t)
            last[r] = t
            if len(toks[r]) >= c.opts[r]["max_tokens"]:
                live[r] = False
        step += 1
    with open(OUT, "w") as f:
        for r in range(c.n):
            f.write(json.dumps({"row": r, "toks": toks[r], "stopped": stopped[r]}) + "\n")
    print(f"wrote {OUT}: {c.n} sequences, {step} steps, {sum(stopped)} stopped by the stop id")


if __name__ == "__main__":
    main()
