"""Writes tests/golden/sampler_golden.npz from the compiled reference sampler.

Run in a container that has the reference tree (it builds oracle/_ref/libvref.so from the
reference's own sources with oracle/Makefile). Every expected id in the fixture is produced by
verbo::Sampler itself (reference src/sampler.cpp), through oracle/ref_shim.cpp:
    python tests/golden/make_golden.py

Fixture layout (numpy .npz, no pickles):
  case{i}_logits  float32[V]        (absent for constant rows: case{i}_fill, case{i}_n)
  case{i}_cfg     SAMPLING 1-elem   verbo::Sampling fields
  case{i}_hist    int32[H]          ids accepted before the first pick
  case{i}_run     int32[2]          (n_picks, accept_each)
  case{i}_ids     int32[n_picks]    the reference's picks
  wl{j}_*         the same for rows of the synthetic workloads (logits regenerated from
                  verbo_amd.workloads; wl{j}_sha pins the generator output)
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT))

import oracle as O  # noqa: E402
from verbo_amd import workloads as W  # noqa: E402

OUT = Path(__file__).resolve().parent / "sampler_golden.npz"
SINGLE = Path(__file__).resolve().parent / "single_draws_golden.npz"


def cfg_arr(c):
    return O.params_array([c])


def main():
    O.build(ref=True)
    rng = np.random.default_rng(20261201)
    arrays = {}
    cases = []
    kat = np.array([0.1, 3.0, 2.9, -1.0, 0.0], np.float32)
    # the reference's own KAT inputs (tests/test_core.cpp:454-496), with seeds
    cases += [
        (kat, O.sampling(temp=0.0), [], 4, 0),
        (kat, O.sampling(seed=42, top_k=2, top_p=1.0), [], 400, 0),
        (kat, O.sampling(seed=1, top_k=0, top_p=0.5), [], 100, 0),
        (kat, O.sampling(seed=1, top_k=0, top_p=1.0, min_p=0.5), [], 100, 0),
        (kat, O.sampling(temp=0.0, repeat=2.0), [1], 2, 0),
        (kat, O.sampling(seed=9, repeat=2.0, repeat_last=1), [1, 2, 1], 50, 1),
    ]
    # random cases: every stage, ties, -inf, signed zeros, odd histories
    for t in range(90):
        V = int(rng.choice([1, 2, 3, 5, 17, 64, 100, 257, 401, 1000]))
        scale = float(rng.choice([0.05, 1.0, 3.0, 20.0]))
        lg = rng.normal(0.0, scale, V).astype(np.float32)
        if t % 5 == 0:
            lg = np.round(lg).astype(np.float32)  # many exact ties
        if t % 7 == 0 and V > 3:
            lg[rng.integers(0, V, 2)] = -np.inf
        if t % 11 == 0 and V > 3:
            lg[rng.integers(0, V, 2)] = np.float32(-0.0)
            lg[rng.integers(0, V, 1)] = np.float32(0.0)
        c = O.sampling(
            temp=float(rng.choice([0.0, 0.25, 0.7, 1.0, 1.7])),
            top_k=int(rng.choice([0, 1, 3, 40, max(V - 1, 1), V, V + 5])),
            top_p=float(rng.choice([0.0, 0.3, 0.9, 0.999, 1.0])),
            min_p=float(rng.choice([0.0, 0.0, 0.01, 0.2, 1.5])),
            repeat=float(rng.choice([1.0, 1.1, 0.8, 2.0])),
            repeat_last=int(rng.choice([0, 1, 8, 64, -3])),
            seed=int(rng.integers(1, 1 << 63)),
        )
        H = int(rng.integers(0, 3 * V + 10))
        hist = rng.integers(-3, V + 3, H).astype(np.int32)
        cases.append((lg, c, hist, 12, int(t % 2)))
    # stream pins: equal logits, the pick is ceil(u*V)-1 (top 16 bits of each draw)
    for seed in (1, 42, 0x123456789ABCDEF, (1 << 64) - 1):
        cases.append((("fill", 0.0, 65536), O.sampling(temp=1.0, top_k=0, top_p=1.0, seed=seed), [], 256, 0))

    for i, (lg, c, hist, n, acc) in enumerate(cases):
        if isinstance(lg, tuple):
            _, fill, V = lg
            row = np.full(V, fill, np.float32)
            arrays[f"case{i}_fill"] = np.array([fill], np.float32)
            arrays[f"case{i}_n"] = np.array([V], np.int32)
        else:
            row = lg
            arrays[f"case{i}_logits"] = row
        ids = O.ref_sampler_run(row, c, hist, n_picks=n, accept_each=bool(acc))
        arrays[f"case{i}_cfg"] = cfg_arr(c)
        arrays[f"case{i}_hist"] = np.asarray(hist, np.int32)
        arrays[f"case{i}_run"] = np.array([n, acc], np.int32)
        arrays[f"case{i}_ids"] = ids
    arrays["n_cases"] = np.array([len(cases)], np.int32)

    # workload rows: 4 rows of each workload, the workload's own parameters, a nonzero seed
    wl = 0
    for name in W.WORKLOADS:
        w = W.make(name, rows=4)
        for r in range(w.B):
            p = w.row_params(r).copy()
            if p["seed"] == 0:
                p["seed"] = 1000 + r
            p["repeat_last"] = 0
            c = O.Sampling(*[p[f].item() for f in O.SAMPLING_DTYPE.names])
            hist = w.hist[w.hist_off[r]:w.hist_off[r + 1]]
            n = 24 if name == "single" else 3
            ids = O.ref_sampler_run(w.logits[r], c, hist, n_picks=n, accept_each=False)
            arrays[f"wl{wl}_name"] = np.array([W.WORKLOADS.index(name)], np.int32)
            arrays[f"wl{wl}_row"] = np.array([r], np.int32)
            arrays[f"wl{wl}_sha"] = np.frombuffer(hashlib.sha256(w.logits[r].tobytes()).digest(), np.uint8)
            arrays[f"wl{wl}_cfg"] = cfg_arr(c)
            arrays[f"wl{wl}_run"] = np.array([n, 0], np.int32)
            arrays[f"wl{wl}_ids"] = ids
            wl += 1
    arrays["n_wl"] = np.array([wl], np.int32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(cases)} cases, {wl} workload rows)")


def single_draws(n=10000):
    """The single-row workload's 10,000 consecutive draws (1 x 49152, seed 42, its 64-id history
    accepted first, no accept between draws) from the compiled reference Sampler: ids[n], the
    row's sha256 (the logits are regenerated from verbo_amd.workloads) and its parameters."""
    w = W.make("single")
    p = w.params[0].copy()
    c = O.Sampling(*[p[f].item() for f in O.SAMPLING_DTYPE.names])
    ids = O.ref_sampler_run(w.logits[0], c, w.hist, n_picks=n, accept_each=False)
    np.savez_compressed(SINGLE, ids=ids.astype(np.int32), cfg=cfg_arr(c),
                        sha=np.frombuffer(hashlib.sha256(w.logits[0].tobytes()).digest(), np.uint8))
    print(f"wrote {SINGLE} ({n} draws, {len(np.unique(ids))} distinct ids)")


if __name__ == "__main__":
    main()
    single_draws()
