"""Pins the oracle (oracle/vsmp_oracle.c) before it is trusted as the GPU checker.

- the reference's own sampler KATs (tests/test_core.cpp:454-496);
- the reference's picks recorded from the compiled reference (tests/golden/, make_golden.py);
- the compiled reference itself, when oracle/_ref is built here;
- published SplitMix64 vectors and closed forms (inverse-CDF walk, softmax mass, min-p and
  top-p cuts) recomputed with numpy by a different method (full lexsort, vectorised cumsum).
"""
import hashlib

import numpy as np
import pytest

KAT = np.array([0.1, 3.0, 2.9, -1.0, 0.0], np.float32)


def test_reference_kats(oracle):
    O = oracle
    # greedy (tests/test_core.cpp:455-458)
    assert O.pick(KAT, O.sampling(temp=0.0))[0] == 1
    # same seed -> same stream, draws in {1,2}, P(1) ~ .536 (:459-471)
    c = O.sampling(seed=42, top_k=2, top_p=1.0)
    a = O.sampler_run(KAT, c, n_picks=400)
    b = O.sampler_run(KAT, c, n_picks=400)
    assert (a == b).all() and set(a.tolist()) <= {1, 2}
    assert 150 < int((a == 1).sum()) < 300
    # top-p .5 -> always 1 (:472-477)
    assert (O.sampler_run(KAT, O.sampling(seed=1, top_k=0, top_p=0.5), n_picks=100) == 1).all()
    # min-p .5 -> {1,2} (:478-487)
    x = O.sampler_run(KAT, O.sampling(seed=1, top_k=0, top_p=1.0, min_p=0.5), n_picks=100)
    assert set(x.tolist()) <= {1, 2}
    # penalty (:488-495)
    assert O.pick(KAT, O.sampling(temp=0.0, repeat=2.0), hist=[1])[0] == 2
    assert O.pick(KAT, O.sampling(temp=0.0, repeat=2.0), hist=[])[0] == 1


def test_splitmix_published_vectors(oracle):
    # SplitMix64 (Steele, Lea, Flood 2014) seeded with 1234567: the first outputs of the
    # published C implementation.
    import ctypes

    s = ctypes.c_uint64(1234567)
    got = [oracle.load_oracle().vo_splitmix(ctypes.byref(s)) for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def test_counter_u_is_the_splitmix_stream(oracle):
    from verbo_amd import workloads as W

    for seed in (0, 7, 1 << 63):
        want = (W.splitmix(seed, 0, 50) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        got = np.array([oracle.counter_u(seed, c) for c in range(50)])
        assert (got == want).all()


def test_golden_reference_picks(oracle, golden):
    """Every pick the compiled reference recorded is reproduced by the oracle's restatement
    (seeding, xorshift stream, accept trimming and the whole pick pipeline)."""
    bad = []
    for c in golden:
        if "sha" in c:
            assert hashlib.sha256(c["logits"].tobytes()).digest() == c["sha"], f"{c['name']}: generator drifted"
        got = oracle.sampler_run(c["logits"], c["cfg"], c["hist"], n_picks=c["n"], accept_each=c["accept"])
        if not (got == c["ids"]).all():
            bad.append(c["name"])
    assert not bad, bad


def test_stream_pins_reveal_draws(oracle, golden):
    """Equal logits make the pick ceil(u*V)-1: the reference's picks give the top 16 bits of
    each draw, which the oracle's xorshift128+ restatement must reproduce."""
    pins = [c for c in golden if c["logits"].size == 65536 and (c["logits"] == 0).all()]
    assert len(pins) == 4
    for c in pins:
        u = oracle.reference_stream(c["cfg"].seed, c["n"])
        assert (np.ceil(u * 65536) - 1 == c["ids"]).all()


@pytest.mark.skipif(not __import__("oracle").ref_available(), reason="compiled reference not built here")
def test_oracle_matches_compiled_reference(oracle):
    rng = np.random.default_rng(7)
    for t in range(200):
        V = int(rng.integers(1, 2500))
        lg = rng.normal(0, rng.uniform(0.1, 6.0), V).astype(np.float32)
        if t % 4 == 0:
            lg = np.round(lg * 2).astype(np.float32)
        c = oracle.sampling(temp=float(rng.choice([0.0, 0.5, 1.0, 2.0])), top_k=int(rng.choice([0, 2, 50, 3000])),
                            top_p=float(rng.choice([0.0, 0.8, 0.95, 1.0])), min_p=float(rng.choice([0, .05, .3])),
                            repeat=float(rng.choice([1.0, 1.3, 0.7])), repeat_last=int(rng.choice([0, 4, 64])),
                            seed=int(rng.integers(1, 1 << 62)))
        hist = rng.integers(-2, V + 2, int(rng.integers(0, 400)))
        for acc in (False, True):
            a = oracle.sampler_run(lg, c, hist, n_picks=8, accept_each=acc)
            b = oracle.ref_sampler_run(lg, c, hist, n_picks=8, accept_each=acc)
            assert (a == b).all(), (t, acc)


def _penalised(lg, hist, repeat, repeat_last):
    """Penalty by numpy: window, de-duplicate, in range, fp32 divide / multiply."""
    v = lg.astype(np.float32).copy()
    h = np.asarray(hist, np.int64)
    if repeat != np.float32(1.0) and h.size:
        if repeat_last > 0 and h.size > repeat_last:
            h = h[h.size - repeat_last:]
        h = np.unique(h)
        h = h[(h >= 0) & (h < v.size)]
        r = np.float32(repeat)
        x = v[h]
        v[h] = np.where(x > 0, x / r, x * r).astype(np.float32)
    return v


def _sorted_ids(v):
    return np.lexsort((np.arange(v.size), -v.astype(np.float64)))


def test_topk_order_and_penalty_brute_force(oracle):
    rng = np.random.default_rng(3)
    for t in range(60):
        V = int(rng.integers(2, 600))
        lg = np.round(rng.normal(0, 3, V) * (1 if t % 2 else 4)).astype(np.float32) / 4
        hist = rng.integers(-2, V + 2, int(rng.integers(0, 50)))
        rep = float(rng.choice([1.0, 1.5, 0.5]))
        rl = int(rng.choice([0, 5, 64]))
        k = int(rng.choice([1, 5, V]))
        c = oracle.sampling(temp=1.0, top_k=k, top_p=1.0, min_p=0.0, repeat=rep, repeat_last=rl, seed=1)
        _, info, cand, _, _ = oracle.pick(lg, c, hist, u=0.5, cand_cap=V)
        order = _sorted_ids(_penalised(lg, hist, np.float32(rep), rl))
        kk = k if 0 < k < V else V
        assert info.k == kk and info.keep == kk
        assert (cand == order[:kk]).all()
        g = oracle.pick(lg, oracle.sampling(temp=0.0, repeat=rep, repeat_last=rl), hist)[0]
        assert g == order[0]


def test_penalised_ids_and_last_id_brute_force(oracle):
    """The oracle's penalised-id list (ascending distinct in-range ids of the window, none when
    repeat == 1) and its draw set's last id, which the GPU's diagnostics are compared with, against
    a brute force: the ids whose value the penalty changed, and the keep-th id of a full sort.
    Batched rows (vo_pick_rows) give the same lists as single picks."""
    rng = np.random.default_rng(13)
    rows = []
    for t in range(40):
        V = 97
        lg = (rng.normal(0, 2, V).astype(np.float32) + 0.25).astype(np.float32)
        lg[lg == 0] = 0.5  # the penalty leaves 0 unchanged; keep every value visibly penalisable
        hist = rng.integers(-3, V + 3, int(rng.integers(0, 80)))
        rep = float(rng.choice([1.0, 1.3, 0.7]))
        rl = int(rng.choice([0, 7, 64, -1]))
        c = oracle.sampling(temp=0.9, top_k=int(rng.choice([0, 5, 30])), top_p=float(rng.choice([0.6, 1.0])),
                            min_p=0.0, repeat=rep, repeat_last=rl, seed=1)
        _, info, cand, _, pen = oracle.pick(lg, c, hist, u=0.4, cand_cap=V, pen_cap=V)
        changed = np.flatnonzero(_penalised(lg, hist, np.float32(rep), rl) != lg)
        assert pen.tolist() == changed.tolist() and info.n_pen == changed.size, t
        order = _sorted_ids(_penalised(lg, hist, np.float32(rep), rl))
        assert info.last_id == order[info.keep - 1] == cand[info.keep - 1]
        rows.append((lg, c, hist, pen, info.last_id))
    lg = np.stack([r[0] for r in rows])
    params = oracle.params_array([r[1] for r in rows])
    off = np.concatenate([[0], np.cumsum([len(r[2]) for r in rows])]).astype(np.int32)
    flat = np.concatenate([r[2] for r in rows]).astype(np.int32)
    _, infos, _, _, pens = oracle.pick_rows(lg, params, flat, off, np.full(len(rows), 0.4), pen_cap=97)
    for r, row in enumerate(rows):
        assert pens[r].tolist() == row[3].tolist() and infos["last_id"][r] == row[4]


def test_inverse_cdf_closed_forms(oracle):
    rng = np.random.default_rng(5)
    # equal logits: the draw is ceil(u*V)-1
    V = 1000
    c = oracle.sampling(temp=1.0, top_k=0, top_p=1.0)
    for u in rng.uniform(0, 1, 200):
        assert oracle.pick(np.zeros(V, np.float32), c, u=u)[0] == max(int(np.ceil(u * V)) - 1, 0)
    # softmax mass: a uniform grid of u lands on each id in proportion to its probability
    lg = rng.normal(0, 1.5, 40).astype(np.float32)
    T = 0.8
    v = lg.astype(np.float64)
    order = _sorted_ids(lg)
    p = np.exp((np.float32(lg[order] - lg.max())).astype(np.float64) / T)
    p /= p.sum()
    N = 20000
    got = np.bincount([oracle.pick(lg, oracle.sampling(temp=T, top_k=0, top_p=1.0), u=(j + 0.5) / N)[0]
                       for j in range(N)], minlength=lg.size)
    assert np.abs(got[order] - N * p).max() <= 1.0 + 1e-9
    del v


def test_minp_topp_cuts_closed_form(oracle):
    rng = np.random.default_rng(11)
    for t in range(80):
        V = int(rng.integers(5, 400))
        lg = rng.normal(0, 2.0, V).astype(np.float32)
        T = float(rng.uniform(0.3, 1.5))
        mp = float(rng.choice([0.0, 0.02, 0.1, 0.5]))
        tp = float(rng.choice([0.5, 0.9, 0.99]))
        c = oracle.sampling(temp=T, top_k=0, top_p=tp, min_p=mp)
        _, info, _, _, _ = oracle.pick(lg, c, u=0.3)
        s = lg[_sorted_ids(lg)]
        pr = np.exp((s - s[0]).astype(np.float64) / np.float64(np.float32(T)))
        keep = V
        if mp > 0:
            keep = max(1, int((pr >= np.float64(np.float32(mp))).sum()))
        assert info.keep_minp == keep
        acc = np.cumsum(pr / pr.sum())
        hit = np.flatnonzero(acc[:keep] >= np.float64(np.float32(tp)))
        want = min(keep, int(hit[0]) + 1) if hit.size else keep
        if info.topp_margin > 1e-12:
            assert info.keep == want, (t, info.keep, want)


def test_single_workload_10000_draws(oracle):
    """The oracle's Sampler run reproduces the compiled reference's 10,000 consecutive draws on the
    single-row workload (tests/golden/single_draws_golden.npz: seed 42, history accepted, no accept
    between draws)."""
    from pathlib import Path

    from verbo_amd import workloads as W

    z = np.load(Path(__file__).resolve().parent / "golden" / "single_draws_golden.npz", allow_pickle=False)
    w = W.make("single")
    assert hashlib.sha256(w.logits[0].tobytes()).digest() == bytes(z["sha"])
    c = z["cfg"][0]
    cfg = oracle.Sampling(*[c[f].item() for f in oracle.SAMPLING_DTYPE.names])
    ids = oracle.sampler_run(w.logits[0], cfg, w.hist, n_picks=int(z["ids"].size))
    assert (ids == z["ids"]).all()
