"""Records the continuous-batching golden: every request of verbo_amd.workloads.ServeCase decoded
alone by its own reference verbo::Sampler (the reference's src/sampler.cpp compiled from its sources
into oracle/_ref/libvref.so), in verbo::generate's order (reference src/sampler.cpp:111-181: the
prompt accepted first; per step pick, a stop id ends the sequence unaccepted, any other id is
accepted, until max_tokens), each step's logits those of the request's own step.

    make -C oracle ref && python tests/golden/make_serve_golden.py

Writes tests/golden/serve_golden.jsonl: per request its tokens and whether a stop id ended it.
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT))

import oracle as O  # noqa: E402
from verbo_amd.workloads import ServeCase  # noqa: E402

OUT = Path(__file__).resolve().parent / "serve_golden.jsonl"


def main():
    c = ServeCase()
    rows = []
    for j in range(c.n):
        o = c.opts[j]
        s = O.RefSampler(O.sampling(temp=o["temp"], top_k=o["top_k"], top_p=o["top_p"], min_p=o["min_p"],
                                    repeat=o["repeat"], repeat_last=c.repeat_last[j], seed=o["seed"]))
        for t in c.prompts[j]:
            s.accept(int(t))
        toks, stopped, last = [], False, -1
        t = 0
        while len(toks) < o["max_tokens"]:
            tok = s.pick(c.logits([j], [t], [last])[0])
            t += 1
            if tok in c.stop_ids:
                stopped = True
                break
            s.accept(tok)
            toks.append(tok)
            last = tok
        rows.append({"req": j, "toks": toks, "stopped": stopped})
    with open(OUT, "w") as f:
        for r in rows:
            f.write(json.dumps(r) + "\n")
    print(f"wrote {OUT}: {c.n} requests, {sum(r['stopped'] for r in rows)} stopped by the stop id, "
          f"{sum(len(r['toks']) for r in rows)} tokens")


if __name__ == "__main__":
    main()
