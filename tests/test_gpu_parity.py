"""Parity of the HIP sampler with the reference, through the C ABI, on an MI355X.

Mirrors the reference's sampler tests (tests/test_core.cpp:454-496) and extends them: golden
picks recorded from the compiled reference, every stage against the oracle on seeded random
batches, all five workloads (reduced and full size), the three draw modes and the edge cases.
"""
import numpy as np
import pytest

import oracle as O
import verbo_amd as V
from helpers import Run, csr, log, mode_ctx
from verbo_amd import workloads as W

pytestmark = pytest.mark.gpu

KAT = np.array([0.1, 3.0, 2.9, -1.0, 0.0], np.float32)


@pytest.fixture(params=["slices", "rows", "split"])
def mode(request):
    """Each decomposition on the same inputs: slices + merge, one workgroup per row, and (for
    greedy and small-k batches with shared parameters; other batches take the default) rows cut
    into parts finished by their last part. A context reads VSMP_MODE when it is created."""
    return request.param


@pytest.fixture
def ctx(request):
    """A context in the test's decomposition mode (the planner's choice when it has none)."""
    import torch

    assert torch.cuda.is_available(), "the gpu tests need a ROCm device"
    m = request.getfixturevalue("mode") if "mode" in request.fixturenames else None
    return mode_ctx(m)


def test_reference_kats_on_gpu():
    """tests/test_core.cpp:454-496 through the drop-in verbo::Sampler."""
    log("kats")
    assert V.Sampler(temp=0.0).pick(KAT) == 1
    a, b = V.Sampler(seed=42, top_k=2, top_p=1.0), V.Sampler(seed=42, top_k=2, top_p=1.0)
    c1 = 0
    for _ in range(400):
        x = a.pick(KAT)
        assert x == b.pick(KAT)
        assert x in (1, 2)
        c1 += x == 1
    assert 150 < c1 < 300
    sp = V.Sampler(seed=1, top_k=0, top_p=0.5)
    assert all(sp.pick(KAT) == 1 for _ in range(100))
    sm = V.Sampler(seed=1, top_k=0, top_p=1.0, min_p=0.5)
    assert all(sm.pick(KAT) in (1, 2) for _ in range(100))
    sr = V.Sampler(temp=0.0, repeat=2.0)
    sr.accept(1)
    assert sr.pick(KAT) == 2
    sr.reset()
    assert sr.pick(KAT) == 1
    with pytest.raises(V.VsmpError):
        V.Sampler().pick(np.zeros(0, np.float32))


def test_golden_reference_sequences(golden):
    """The drop-in Sampler on the GPU replays every pick the compiled reference recorded:
    same seeds, histories, accepts -> the same ids."""
    bad = []
    for c in golden:
        log("golden", c["name"], c["logits"].size)
        s = V.Sampler(V.Params(*[getattr(c["cfg"], f) for f, _ in O.Sampling._fields_]))
        for t in c["hist"]:
            s.accept(int(t))
        got = []
        for _ in range(c["n"]):
            got.append(s.pick(c["logits"]))
            if c["accept"]:
                s.accept(got[-1])
        if got != c["ids"].tolist():
            bad.append((c["name"], got[:8], c["ids"][:8].tolist()))
    assert not bad, bad


def _random_batch(rng, B, Vv, per_row=True, ties=False):
    scale = rng.choice([0.05, 1.0, 3.0, 10.0])
    lg = rng.normal(0, scale, (B, Vv)).astype(np.float32)
    if ties:
        lg = np.round(lg).astype(np.float32)
    n = B if per_row else 1
    p = np.zeros(n, V.SAMPLING_DTYPE)
    p["temp"] = rng.choice([0.0, 0.3, 0.7, 1.0, 1.6], n)
    p["top_k"] = rng.choice([0, 1, 2, 40, 256, 257, 1000, Vv - 1, Vv + 3], n)
    p["top_p"] = rng.choice([0.0, 0.5, 0.9, 0.99, 1.0], n)
    p["min_p"] = rng.choice([0.0, 0.0, 0.05, 0.3, 1.5], n)
    p["repeat"] = rng.choice([1.0, 1.2, 0.8], n)
    p["repeat_last"] = rng.choice([0, 3, 64, -1], n)
    p["seed"] = rng.integers(1, 1 << 62, n)
    hists = [rng.integers(-2, Vv + 2, int(rng.integers(0, 300))) for _ in range(B)]
    h, off = csr(hists)
    return lg, p, h, off


@pytest.mark.parametrize("seed", range(6))
def test_random_batches_match_oracle(ctx, mode, seed):
    rng = np.random.default_rng(100 + seed)
    for Vv in (1, 3, 5, 64, 257, 1023, 4099, 20000):
        B = int(rng.integers(1, 40))
        lg, p, h, off = _random_batch(rng, B, Vv, per_row=bool(seed % 2 == 0), ties=seed % 3 == 0)
        log("random", mode, seed, B, Vv)
        run = Run(ctx, lg, p, h, off, cand_cap=256)
        run.report()


def test_edge_rows(ctx, mode):
    Vv = 777
    rows = []
    r = np.zeros(Vv, np.float32)
    rows.append(r)                                  # all equal
    r = np.full(Vv, -np.inf, np.float32)
    r[5] = 1.0
    rows.append(r)                                  # one finite value
    r = np.zeros(Vv, np.float32)
    r[::2] = -0.0
    r[100] = r[200] = 3.0
    rows.append(r)                                  # signed zeros, exact tie at the max
    r = np.arange(Vv, dtype=np.float32)
    rows.append(r)                                  # ascending: the adversarial order
    r = -np.arange(Vv, dtype=np.float32)
    rows.append(r)                                  # descending
    r = np.random.default_rng(0).normal(0, 1, Vv).astype(np.float32)
    r[300:] = 2.5
    rows.append(r)                                  # a large tie group near the top
    lg = np.stack(rows)
    for temp, top_k, top_p, min_p in [(0.0, 40, 0.9, 0.0), (0.7, 40, 0.9, 0.0), (1.0, 0, 1.0, 0.0),
                                      (1.0, 0, 0.5, 0.0), (0.5, 600, 0.95, 0.1), (2.0, 3, 0.99, 2.0),
                                      (1e-3, 0, 0.9, 0.0), (1.0, Vv, 0.0, 0.0)]:
        p = V.params_array(n=1, temp=temp, top_k=top_k, top_p=top_p, min_p=min_p, repeat=1.3, repeat_last=0,
                           seed=3)
        hists = [[5, 5, 100, -1, Vv, 700]] * len(rows)
        h, off = csr(hists)
        log("edge", mode, temp, top_k, top_p, min_p)
        for u in (0.0, 0.37, 1.0 - 2.0 ** -53):
            Run(ctx, lg, p, h, off, u=np.full(len(rows), u), cand_cap=64).report()


def test_maximum_first_index(ctx, mode):
    """The general path's row maximum and its first index (src/sampler.cpp:72-78: value descending,
    then index ascending; -0 == +0), where one thread meets the maximum in several of its 16-byte
    groups (at 512 and 1024 threads a thread's groups lie 2,048 and 4,096 elements apart), in a lone
    element past the last whole group, and among -inf. u = 0 draws the first element of the order."""
    Vv = 20001
    rng = np.random.default_rng(77)
    base = -1.0 - rng.random(Vv).astype(np.float32)
    rows = []
    r = base.copy(); r[4] = -0.0; r[2052] = 0.0; r[4100] = 0.0
    rows.append(r)                                  # -0 first, +0 later in the same thread's groups
    r = base.copy(); r[6] = 0.0; r[2054] = -0.0; r[4102] = -0.0; r[3] = -0.0
    rows.append(r)                                  # -0 ahead of +0 in another thread's group
    r = base.copy(); r[Vv - 1] = 2.0; r[Vv - 2] = 2.0
    rows.append(r)                                  # the maximum twice in the ragged tail
    r = base.copy(); r[Vv - 1] = 2.0; r[9] = 2.0; r[2057] = 2.0
    rows.append(r)                                  # ... and earlier in whole groups
    r = np.full(Vv, -np.inf, np.float32); r[[4097, 5, 2053]] = [0.0, -0.0, 0.0]
    rows.append(r)                                  # -inf around signed zeros
    r = base.copy(); r[::3] = 1.5
    rows.append(r)                                  # the maximum in every thread's first group
    lg = np.stack(rows)
    for temp, top_k, top_p, min_p in [(1.0, 0, 0.9, 0.0), (0.5, 600, 0.95, 0.05), (1.0, 0, 0.5, 0.5)]:
        p = V.params_array(n=1, temp=temp, top_k=top_k, top_p=top_p, min_p=min_p, repeat=1.0, repeat_last=0,
                           seed=11)
        log("maximum first index", mode, temp, top_k, top_p, min_p)
        for u in (0.0, 0.5):
            Run(ctx, lg, p, None, None, u=np.full(len(rows), u), cand_cap=8).report()
    # the same rows penalised: a penalised maximum gives way to the next value
    hists = [[4, 2052, 6, Vv - 1, 9, 5, 0]] * len(rows)
    p = V.params_array(n=1, temp=1.0, top_k=0, top_p=0.9, min_p=0.0, repeat=1.3, repeat_last=0, seed=11)
    log("maximum first index, penalised", mode)
    Run(ctx, lg, p, *csr(hists), u=np.zeros(len(rows)), cand_cap=8).report()


def test_general_full_buckets(ctx, mode):
    """The general path on rows where one level-0 bucket holds thousands of elements (its histogram
    adds all meet on one address): one value repeated 7,990, 8,100, 9,000 and 70,000 times among
    N(0, 1) values, with top-p, a capped row (temp .02), a top-k cut and min-p."""
    rng = np.random.default_rng(515)
    rows = []
    for Vv, n_eq in ((30000, 7990), (30000, 8100), (30000, 9000), (151936, 70000)):
        r = rng.normal(0, 1, Vv).astype(np.float32)
        pos = rng.choice(Vv, n_eq, replace=False)
        r[pos] = np.float32(0.25)
        rows.append(r)
    for r in rows:
        Vv = r.size
        lg = r[None, :]
        for temp, top_k, top_p, min_p in [(1.0, 0, 0.9, 0.0), (0.02, 0, 0.95, 0.0), (0.8, 1000, 0.9, 0.0),
                                          (1.0, 0, 0.99, 0.01)]:
            p = V.params_array(n=1, temp=temp, top_k=top_k, top_p=top_p, min_p=min_p, repeat=1.0, repeat_last=0,
                               seed=5)
            log("full buckets", mode, Vv, temp, top_k, top_p, min_p)
            for u in (0.3, 0.999):
                Run(ctx, lg, p, None, None, u=np.full(1, u), cand_cap=16).report()


def test_no_history_and_padded_rows(ctx, mode):
    rng = np.random.default_rng(9)
    lg = rng.normal(0, 2, (7, 1001)).astype(np.float32)
    p = V.params_array(n=1, temp=0.9, top_k=50, top_p=0.9, min_p=0.02, seed=5)
    log("padded ld")
    Run(ctx, lg, p, None, None, ld=1024, cand_cap=50).report()
    Run(ctx, lg, p, *csr([[]] * 7), ld=1100, cand_cap=50).report()


@pytest.mark.parametrize("name", ["single", "greedy", "peaked", "wide", "mixed"])
def test_workloads_reduced(ctx, mode, name):
    w = W.make(name, rows=32)
    log("workload", mode, name, w.B, w.V)
    run = Run(ctx, w.logits, w.params, w.hist, w.hist_off, cand_cap=256)
    n, nm = run.report()
    log(f"  {run.counts}")
    assert nm == 0


@pytest.mark.parametrize("name", ["greedy", "peaked", "wide", "mixed"])
def test_workloads_full_size(ctx, name):
    """Every row of the four batched workloads at full size, every diagnostic compared; the
    draws within 1e-6 of a CDF boundary are counted and must still pick the oracle's id."""
    w = W.make(name)
    log("workload full", name, w.B, w.V)
    run = Run(ctx, w.logits, w.params, w.hist, w.hist_off, cand_cap=128)
    n, nm = run.report()
    log(f"  {run.counts}")
    assert nm == 0


def test_draw_modes(ctx, mode):
    import torch

    rng = np.random.default_rng(4)
    B, Vv = 48, 5000
    lg = rng.normal(0, 2, (B, Vv)).astype(np.float32)
    p = np.zeros(B, V.SAMPLING_DTYPE)
    p["temp"] = np.where(np.arange(B) % 4 == 0, 0.0, 0.8)
    p["top_k"] = np.where(np.arange(B) % 3 == 0, 0, 40)
    p["top_p"], p["min_p"], p["repeat"], p["repeat_last"] = 0.9, 0.0, 1.0, 64
    p["seed"] = np.arange(1, B + 1)
    d = torch.from_numpy(lg).cuda()
    dp = V.to_device_params(p)
    # counter mode: u = output `counter` of the row's SplitMix64 stream
    for counter in (0, 5):
        log("counter mode", counter)
        ids = ctx.pick_batch(d, dp, u_mode=V.U_COUNTER, counter=counter).cpu().numpy()
        u = np.array([O.counter_u(int(p["seed"][r]), counter) for r in range(B)])
        o = O.pick_rows(lg, p, u=u)[0]
        assert (ids == o).all()
    # xorshift mode: the reference stream of each row, advanced once per non-greedy pick
    st = np.zeros((B, 2), np.uint64)
    for r in range(B):
        s = O.rng_seed(int(p["seed"][r]))
        st[r] = [s[0], s[1]]
    dst = torch.from_numpy(st.view(np.int64).copy()).cuda()
    for step in range(3):
        log("xorshift mode", step)
        ids = ctx.pick_batch(d, dp, u_mode=V.U_XORSHIFT, rng_state=dst).cpu().numpy()
        u = np.zeros(B)
        for r in range(B):
            if p["temp"][r] > 0:
                s = (O.ctypes.c_uint64 * 2)(int(st[r, 0]), int(st[r, 1]))
                u[r] = O.rng_unit(s)
                st[r] = [s[0], s[1]]
        o = O.pick_rows(lg, p, u=u)[0]
        assert (ids == o).all()
        assert (dst.cpu().numpy().view(np.uint64) == st).all()


def test_bad_arguments(ctx):
    import torch

    d = torch.zeros((2, 8), device="cuda")
    p = V.Params()
    with pytest.raises(V.VsmpError, match="u is required"):
        ctx.pick_batch(d, p, u_mode=V.U_SUPPLIED)
    with pytest.raises(V.VsmpError, match="ld must be"):
        ctx.pick_batch(torch.zeros((2, 16), device="cuda")[:, :7].contiguous().as_strided((2, 7), (7, 1)), p)
    with pytest.raises(V.VsmpError, match="aligned"):
        ctx.pick_batch(torch.zeros(40, device="cuda")[1:33].view(2, 16), p)
    with pytest.raises(V.VsmpError, match="rng_state"):
        ctx.pick_batch(d, p, u_mode=V.U_XORSHIFT)


def test_counter_seeds_with_shared_params(ctx, mode):
    """Shared parameters: row r draws output `counter` of the stream seeded with seed + r."""
    import torch

    w = W.make("peaked", rows=40)
    p = w.params[0]
    d = torch.from_numpy(w.logits).cuda()
    h, ho = torch.from_numpy(w.hist).cuda(), torch.from_numpy(w.hist_off).cuda()
    for counter in (0, 3):
        log("shared counter", mode, counter)
        ids = ctx.pick_batch(d, V.Params(*[p[f].item() for f in V.SAMPLING_DTYPE.names]), h, ho, V.U_COUNTER,
                             counter=counter).cpu().numpy()
        u = np.array([O.counter_u(int(p["seed"]) + r, counter) for r in range(w.B)])
        o = O.pick_rows(w.logits, w.params, w.hist, w.hist_off, u)[0]
        assert (ids == o).all()


def _general_batch(rng, kind, B=24, Vv=30000):
    """Rows that take the general path (top-k off) and one of its pass plans."""
    p = np.zeros(B, V.SAMPLING_DTYPE)
    p["top_k"] = 0
    p["repeat"] = 1.0
    p["seed"] = rng.integers(1, 1 << 62, B)
    hists = [[] for _ in range(B)]
    if kind == "flat":  # the cut's bucket bounds the draw's: one shared pass
        lg = rng.normal(0, 0.5, (B, Vv))
        p["temp"] = 1.0
        p["top_p"] = rng.choice([0.9, 0.95, 0.99], B)
    elif kind == "minp":  # a few spikes hold the min-p prefix: collected whole
        lg = rng.normal(0, 2.0, (B, Vv))
        for r in range(B):
            lg[r, rng.integers(0, Vv, 8)] += 6.0 + 2.0 * rng.random(8)
        p["temp"] = rng.choice([0.5, 0.7, 1.0], B)
        p["top_p"] = rng.choice([0.8, 0.9, 1.0], B)
        p["min_p"] = rng.choice([0.05, 0.1], B)
        p["repeat"] = 1.2
        hists = [rng.integers(0, Vv, int(rng.integers(0, 200))) for _ in range(B)]
    elif kind == "minp_large":  # min-p prefixes of thousands: top-p may cut inside them, or cannot
        lg = rng.normal(0, 0.5, (B, Vv))
        p["temp"] = 0.25
        p["min_p"] = rng.choice([0.005, 0.008, 0.012], B)
        p["top_p"] = np.where(np.arange(B) % 2 == 0, 0.3, 0.995)
    elif kind == "minp_overflow":  # capped rows whose tiny min-p threshold keeps some of the overflow
        # bucket (64 to 69 temp below the maximum): the main pass cannot collect those, and a pass
        # of its own collects the prefix
        lg = np.full((B, Vv), -1e4)
        for r in range(B):
            lg[r, rng.integers(0, Vv, 300)] = rng.uniform(-66.0, -40.0, 300)
            lg[r, rng.integers(0, Vv)] = 0.0
        p["temp"] = 1.0
        p["min_p"] = 1e-30
        p["top_p"] = rng.choice([0.9, 1.0], B)
    elif kind == "cold":  # the buckets stop far short of the minimum: the overflow bucket holds most rows
        lg = rng.normal(0, 2.0, (B, Vv))
        p["temp"] = rng.choice([0.005, 0.02, 0.05], B)
        p["top_p"] = rng.choice([0.95, 1.0], B)
    else:  # general and small-k rows interleaved, per-row parameters: workgroups renumber the general rows
        lg = rng.normal(0, 1.5, (B, Vv))
        p["temp"] = rng.choice([0.0, 0.6, 1.1], B)
        p["top_k"] = rng.choice([0, 0, 40, 300], B)
        p["top_p"] = rng.choice([0.9, 1.0], B)
        p["min_p"] = rng.choice([0.0, 0.05], B)
        p["repeat"] = rng.choice([1.0, 1.3], B)
        hists = [rng.integers(0, Vv, int(rng.integers(0, 500))) for _ in range(B)]
    h, off = csr(hists)
    return lg.astype(np.float32), p, h, off


@pytest.mark.parametrize("kind", ["flat", "minp", "minp_large", "minp_overflow", "cold", "interleaved"])
def test_general_path_pass_plans(ctx, mode, kind):
    rng = np.random.default_rng({"flat": 11, "minp": 12, "minp_large": 15, "minp_overflow": 16, "cold": 13,
                                 "interleaved": 14}[kind])
    lg, p, h, off = _general_batch(rng, kind)
    log("general pass plan", mode, kind)
    run = Run(ctx, lg, p, h, off)
    run.report()
    gen = run.info["path"] == V.PATH_GENERAL
    flags = run.info["flags"][gen]
    if kind == "flat":
        assert (flags & V.FLAG_ONE_PASS).mean() >= 0.5, flags
    if kind in ("minp", "minp_overflow"):
        assert (flags & V.FLAG_MINP_PREFIX).mean() >= 0.5, flags
    if kind == "minp_large":  # prefixes beyond the whole-prefix collection, both top-p outcomes
        keep_m, keep = run.info["keep_minp"][gen], run.info["keep"][gen]
        big = keep_m > 1024
        assert (big & (keep < keep_m)).any() and (big & (keep == keep_m)).any(), (keep_m, keep)
    if kind == "interleaved":
        assert gen.any() and (~gen).any()


def test_general_path_top_p_ties_exact(ctx, mode):
    """Rows of tied logits whose top-p running sum meets top_p at rounding distance: the general
    path's bucket-order sums cannot decide such a cut, so the row is redone in the reference's
    order and sequential sums (k_general_exact). Keep counts and ids equal the oracle's exactly, and
    the redone rows carry VSMP_FLAG_SEQ_CUTS. The logits are all 0, which the penalty leaves as
    they are, so that the rows with a penalised history (half of them) stay tied as well."""
    rng = np.random.default_rng(61)
    for Vv in (4098, 20000, 49152):
        B = 4
        lg = np.zeros((B, Vv), np.float32)
        p = V.params_array(n=B, temp=1.0, top_k=0, top_p=0.5, min_p=0.0, repeat=1.0, repeat_last=0, seed=7)
        p["top_p"] = [0.5, 0.25, 0.75, 0.5]
        p["repeat"] = [1.0, 1.1, 1.0, 1.1]
        p["seed"] = rng.integers(1, 1 << 62, B)
        h, off = csr([list(rng.integers(0, Vv, 100)) if r % 2 else [] for r in range(B)])
        log("top-p ties", mode, Vv)
        run = Run(ctx, lg, p, h, off, cand_cap=128)
        run.report()
        for r in range(B):
            o, g = run.o_info[r], run.info[r]
            assert int(g["keep"]) == int(o["keep"]), (Vv, r, int(g["keep"]), int(o["keep"]))
            assert run.ids[r] == run.o_ids[r], (Vv, r, run.ids[r], run.o_ids[r])
            if o["topp_margin"] < 1e-11:
                assert int(g["flags"]) & V.FLAG_SEQ_CUTS, (Vv, r, int(g["flags"]))


def test_general_path_top_p_ties_sorted(ctx, mode):
    """Near-tie rows that are not flat, so that the exact redo sorts them: a multiple of four
    logits at 0 at random positions, the rest at -1000 (numerators exp(-1000) = 0 in fp64), so the
    top-p running sum meets top_p at rounding distance inside the zeros, which the sort must put
    first in index order. Half the rows carry a penalised history (the penalty takes -1000 to -1200
    and leaves 0). Keep counts and ids equal the oracle's, and rows at a tie carry
    VSMP_FLAG_SEQ_CUTS."""
    rng = np.random.default_rng(62)
    for Vv in (4098, 49152, 151936):
        B = 4
        lg = np.full((B, Vv), -1000.0, np.float32)
        n0 = 4 * (Vv // 10)
        for r in range(B):
            lg[r, rng.choice(Vv, n0, replace=False)] = 0.0
        p = V.params_array(n=B, temp=1.0, top_k=0, top_p=0.5, min_p=0.0, repeat=1.0, repeat_last=0, seed=7)
        p["top_p"] = [0.5, 0.25, 0.75, 0.5]
        p["repeat"] = [1.0, 1.2, 1.0, 1.2]
        p["seed"] = rng.integers(1, 1 << 62, B)
        h, off = csr([list(rng.integers(0, Vv, 100)) if r % 2 else [] for r in range(B)])
        log("top-p ties, sorted redo", mode, Vv)
        run = Run(ctx, lg, p, h, off, cand_cap=128)
        run.report()
        for r in range(B):
            o, g = run.o_info[r], run.info[r]
            assert int(g["keep"]) == int(o["keep"]), (Vv, r, int(g["keep"]), int(o["keep"]))
            assert run.ids[r] == run.o_ids[r], (Vv, r, run.ids[r], run.o_ids[r])
            if o["topp_margin"] < 1e-11:
                assert int(g["flags"]) & V.FLAG_SEQ_CUTS, (Vv, r, int(g["flags"]))
        assert (run.info["flags"] & V.FLAG_SEQ_CUTS).any()


@pytest.mark.parametrize("Vv", [777, 5003, 151936])
def test_general_path_flat_rows(ctx, mode, Vv):
    """Flat general rows (every value the same, as in padding rows), which the main pass takes
    without its histogram atomics: top-k off and 1000, top-p off, .9 and .37, min-p off, .05 and
    1e-30, values 0, -2.5 and 7. Half the rows carry a penalised history. The penalty leaves a row
    of zeros flat, and turns a row of -2.5 into one of two values, which takes the pass; penalised
    rows of 7 are zeros instead, since the penalty would take them off 7. Every comparison of the
    parity bar against the oracle."""
    rng = np.random.default_rng(63)
    combos = [(0, 0.9, 0.0), (0, 1.0, 0.05), (1000, 0.9, 0.0), (1000, 0.37, 1e-30), (0, 0.37, 0.05), (1000, 1.0, 0.0)]
    B = 2 * len(combos) * 3
    lg = np.zeros((B, Vv), np.float32)
    rows = []
    for i, (tk, tp, mp) in enumerate(combos):
        for j, val in enumerate((0.0, -2.5, 7.0)):
            for pen in (False, True):
                r = len(rows)
                lg[r] = val if not (pen and val > 0) else 0.0  # a penalised positive row would not stay flat
                rows.append(dict(temp=0.8, top_k=tk, top_p=tp, min_p=mp, repeat=1.3 if pen else 1.0, repeat_last=0,
                                 seed=int(rng.integers(1, 1 << 62))))
    p = V.params_array(rows)
    h, off = csr([list(rng.integers(0, Vv, 40)) if r % 2 else [] for r in range(B)])
    log("flat general rows", mode, Vv, B)
    run = Run(ctx, lg, p, h, off, cand_cap=64)
    run.report()
    assert (run.info["keep"] == run.o_info["keep"]).all() and (run.ids == run.o_ids).all()


def test_general_path_exp_accuracy(ctx):
    """The general path's fp64 exp (a 64-entry table method) against exp in long double: within
    1.01 ulp over [-745, 0] (the reference's libm exp is within one ulp too), exactly 1 at 0 and 0
    where exp underflows or the argument is -inf."""
    import torch

    rng = np.random.default_rng(21)
    x = np.concatenate([-745.0 * rng.random(300000), -40.0 * rng.random(300000), -rng.random(300000),
                        -0.01 * rng.random(300000), -np.arange(0.0, 745.0, 0.125),
                        np.array([0.0, -0.0, -5e-324, -1e-300, -708.0, -708.5, -744.0])])
    y = ctx.exp_probe(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = np.exp(x.astype(np.longdouble))
    ulp = np.spacing(ref.astype(np.float64)).astype(np.longdouble)
    err = np.abs(y.astype(np.longdouble) - ref) / ulp
    worst = int(np.argmax(err))
    assert err[worst] <= 1.01, (x[worst], y[worst], ref[worst], float(err[worst]))
    assert y[x == 0.0].tolist() == [1.0] * int((x == 0.0).sum())
    special = ctx.exp_probe(torch.tensor([-746.0, -1e5, -np.inf], dtype=torch.float64, device="cuda")).cpu().numpy()
    assert special.tolist() == [0.0, 0.0, 0.0]


@pytest.mark.parametrize("span", [64.0, 20.0, 3.0, 1e-3])
def test_general_path_table_numerator_accuracy(ctx, span):
    """The main pass's numerators (a table over its bucket pairs and a degree-6 polynomial) against
    exp(d / temp) in long double, for the bucket scales of rows whose span is 64 temp (the widest,
    bucket width 1/64 in exponent units), 20, 3 and 1e-3 temp: relative error within
    (2.5 + |x|) * 2^-52, x = d / temp: 2.5 units of the exp itself, and |x| * 2^-52 for the exponent,
    which the path forms as d * (1 / temp) where the reference divides (exact at temp 1, where the
    bound is 2.5 * 2^-52 alone). Elements over the whole span and at every bucket edge (where the
    float bucket index rounds); 1 within an ulp at d = 0."""
    import torch

    rng = np.random.default_rng(31)
    for temp in (1.0, 0.37, 1.9):
        qs = np.float32(4096.0 / (span * temp))
        edges = -(np.arange(4097, dtype=np.float64) / np.float64(qs))
        d = np.concatenate([-np.float64(span * temp) * rng.random(400000), edges, np.nextafter(edges, 0.0),
                            np.nextafter(edges, -np.inf), [0.0, -0.0]]).astype(np.float32)
        d = d[(d <= 0) & (d >= -np.float32(span * temp) * np.float32(0.99999))]
        y = ctx.numer_probe(torch.from_numpy(d).cuda(), temp, float(qs)).cpu().numpy()
        x = d.astype(np.longdouble) / np.longdouble(np.float32(temp))
        ref = np.exp(x)
        rel = np.abs(y.astype(np.longdouble) - ref) / ref / np.longdouble(2.0**-52)
        bound = 2.5 + (np.abs(x) if temp != 1.0 else 0.0)
        worst = int(np.argmax(rel - bound))
        assert rel[worst] <= bound if np.ndim(bound) == 0 else rel[worst] <= bound[worst], \
            (span, temp, float(d[worst]), y[worst], float(ref[worst]), float(rel[worst]))
        assert abs(y[d == 0][0] - 1.0) <= 2.3e-16


@pytest.mark.parametrize("span", [64.0, 20.0, 3.0, 1e-3])
def test_general_path_fixed_point_mass_accuracy(ctx, span):
    """Each element's share of its level-0 bucket's mass (the bucket pair's table value times the
    element's fixed-point term, exp(x - c) rounded to 2^-40) against exp(d / temp) in long double:
    within 5e-13 (relative; the 2^-40 rounding at most 4.6e-13 of it) plus |x| * 2^-52 for the
    exponent's product form, over the same spans, temperatures and bucket edges as the table
    numerators. Parity of the general path's top-p decisions leans on this bound: the near-tie band
    (1e-11 and up) must exceed the prefixes' error, twice 5e-13 at most."""
    import torch

    rng = np.random.default_rng(37)
    for temp in (1.0, 0.37, 1.9):
        qs = np.float32(4096.0 / (span * temp))
        edges = -(np.arange(4097, dtype=np.float64) / np.float64(qs))
        d = np.concatenate([-np.float64(span * temp) * rng.random(400000), edges, np.nextafter(edges, 0.0),
                            np.nextafter(edges, -np.inf), [0.0, -0.0]]).astype(np.float32)
        d = d[(d <= 0) & (d >= -np.float32(span * temp) * np.float32(0.99999))]
        y = ctx.numer_probe(torch.from_numpy(d).cuda(), temp, float(qs), fixed_point=True).cpu().numpy()
        x = d.astype(np.longdouble) / np.longdouble(np.float32(temp))
        ref = np.exp(x)
        rel = np.abs(y.astype(np.longdouble) - ref) / ref
        bound = 5e-13 + (np.abs(x) * np.longdouble(2.0**-52) if temp != 1.0 else 0.0)
        excess = rel - bound
        worst = int(np.argmax(excess))
        assert excess[worst] <= 0, (span, temp, float(d[worst]), y[worst], float(ref[worst]), float(rel[worst]))
        # the rounding is to nearest: the errors are not one-sided
        assert (y > ref).any() and (y < ref).any()


@pytest.mark.parametrize("dmode", ["split", "rows"])
def test_greedy_split_parts(dmode):
    """Greedy batches cut into parts (one launch, the last part of a row writes its id) against the
    oracle and against one workgroup per row: ties of the maximum in different parts (the lowest
    index wins), the maximum itself penalised, parts that end inside a 16-byte group or hold no
    group, consecutive calls reusing the per-row slots, and calls without diagnostics (which fold
    the parts' maxima through one compare-and-swap word per row: two calls in a row at every shape)."""
    import torch

    ctx = mode_ctx(dmode)
    rng = np.random.default_rng(31)
    for B, Vv in [(1, 49152), (3, 1001), (5, 4097), (2, 20001), (17, 151936), (9, 131075), (40, 2052)]:
        lg = rng.normal(0, 3, (B, Vv)).astype(np.float32)
        for r in range(B):
            lg[r, rng.choice(Vv, size=3, replace=False)] = lg[r].max() + 1.0
        hists = [list(rng.integers(-2, Vv + 2, int(rng.integers(0, 600)))) + [int(np.argmax(lg[r]))]
                 for r in range(B)]
        h, off = csr(hists)
        p = V.params_array(n=1, temp=0.0, top_k=40, top_p=0.9, repeat=1.3, repeat_last=0, seed=1)
        log("greedy split", dmode, B, Vv)
        run = Run(ctx, lg, p, h, off)
        run.report()
        assert (run.info["path"] == V.PATH_GREEDY).all()
        for r in range(B):
            hh = np.asarray(hists[r])
            assert run.info["n_pen"][r] == len(np.unique(hh[(hh >= 0) & (hh < Vv)])), r
        buf = torch.zeros((B, (Vv + 3) // 4 * 4), dtype=torch.float32)  # rows padded to a multiple of 4
        buf[:, :Vv] = torch.from_numpy(lg)
        d = buf.cuda()[:, :Vv]
        pr = V.Params(*[p[0][f].item() for f in V.SAMPLING_DTYPE.names])
        for _ in range(2):
            out = ctx.pick_batch(d, pr, torch.from_numpy(h).cuda(), torch.from_numpy(off).cuda())
            torch.cuda.synchronize()
            assert (out.cpu().numpy() == run.o_ids).all(), (B, Vv)


def test_vocabulary_beyond_the_row_kernel(ctx):
    """V above 2^19, where the planner's default is slices: shared and per-row parameters (small-k,
    general and greedy rows), a history, ties at the maximum, against the oracle."""
    rng = np.random.default_rng(41)
    Vv = 600_003
    B = 4
    lg = rng.normal(0, 2, (B, Vv)).astype(np.float32)
    lg[:, rng.choice(Vv, 5, replace=False)] = lg.max() + 1.0
    hists = [list(rng.integers(-3, Vv + 3, 200)) for _ in range(B)]
    h, off = csr(hists)
    for p in (V.params_array(n=1, temp=0.8, top_k=50, top_p=0.95, min_p=0.05, repeat=1.1, repeat_last=0, seed=3),
              V.params_array(n=1, temp=0.0, repeat=1.1, repeat_last=64, seed=3)):
        log("large V shared", Vv, p["temp"][0])
        Run(ctx, lg, p, h, off, cand_cap=64).report()
    p = np.zeros(B, V.SAMPLING_DTYPE)
    p["temp"] = [0.0, 0.7, 1.0, 1.3]
    p["top_k"] = [40, 40, 0, 1000]
    p["top_p"] = [0.9, 0.9, 0.99, 0.5]
    p["min_p"] = [0.0, 0.02, 0.0, 0.0]
    p["repeat"] = [1.2, 1.2, 1.0, 0.9]
    p["repeat_last"] = [0, 16, 64, 0]
    p["seed"] = [11, 12, 13, 14]
    log("large V per row", Vv)
    Run(ctx, lg, p, h, off, cand_cap=64).report()


def test_graph_capture_and_replay(ctx):
    """vsmp_pick_batch captured into a HIP graph (after one eager call has sized the scratch) and
    replayed with new logits and draws copied into the captured buffers between replays: every
    replay equals the eager call on the same inputs, for a greedy batch (split mode), a top-k batch
    (row mode), a general batch (k_general alone) and a batch with per-row parameters mixing top-k
    and general rows (k_rows, and k_general on a stream forked from and joined back to the
    capturing one), all four in one graph."""
    import torch

    rng = np.random.default_rng(51)
    B, Vv = 8, 30000
    cases = [V.params_array(n=1, temp=0.0, repeat=1.2, repeat_last=0, seed=1),
             V.params_array(n=1, temp=0.8, top_k=40, top_p=0.9, min_p=0.02, repeat=1.1, repeat_last=0, seed=1),
             V.params_array(n=1, temp=1.0, top_k=0, top_p=0.95, repeat=1.1, repeat_last=0, seed=1)]
    prm = [V.Params(*[p[0][f].item() for f in V.SAMPLING_DTYPE.names]) for p in cases]
    per_row = V.params_array(n=B, temp=0.9, top_k=40, top_p=0.9, repeat=1.1, repeat_last=0, seed=1)
    per_row["top_k"][::2] = 0
    cases.append(per_row)
    prm.append(V.to_device_params(per_row))
    h, off = csr([list(rng.integers(0, Vv, 100)) for _ in range(B)])
    dh, doff = torch.from_numpy(h).cuda(), torch.from_numpy(off).cuda()
    lg = torch.zeros((B, Vv), dtype=torch.float32, device="cuda")
    u = torch.zeros(B, dtype=torch.float64, device="cuda")
    outs = [torch.zeros(B, dtype=torch.int32, device="cuda") for _ in cases]

    def fill(seed):
        r = np.random.default_rng(seed)
        lg.copy_(torch.from_numpy(r.normal(0, 2, (B, Vv)).astype(np.float32)))
        u.copy_(torch.from_numpy(r.random(B)))

    def eager():
        res = []
        for p in prm:
            res.append(ctx.pick_batch(lg, p, dh, doff, V.U_SUPPLIED, u).cpu().numpy())
        return res

    fill(0)
    eager()  # sizes the scratch outside the capture
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            for p, o in zip(prm, outs):
                ctx.pick_batch(lg, p, dh, doff, V.U_SUPPLIED, u, out=o, stream=st)
    torch.cuda.synchronize()
    for rep in range(5):
        fill(100 + rep)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [o.cpu().numpy() for o in outs]
        want = eager()
        torch.cuda.synchronize()
        log("graph replay", rep)
        for c in range(len(cases)):
            assert (got[c] == want[c]).all(), (rep, c, got[c], want[c])
        lgn = lg.cpu().numpy()
        o_ids = O.pick_rows(lgn, cases[0], h, off, u.cpu().numpy())[0]
        assert (got[0] == o_ids).all()


@pytest.mark.parametrize("dmode", ["split", "rows"])
def test_topk_split_parts(dmode):
    """Small-k batches cut into parts (one launch, the last part merges the parts' sorted lists and
    runs the epilogue) against the oracle, and row mode on the same inputs: ties of the largest
    values in different parts, penalised candidates, k from 1 to 256, min-p and top-p, parts that
    end inside a 16-byte group or hold no group, all three draw modes (the xorshift state advanced
    once per row), candidate lists, and consecutive calls reusing the per-row tickets."""
    import torch

    ctx = mode_ctx(dmode)
    rng = np.random.default_rng(61)
    for B, Vv, k in [(1, 151936, 40), (3, 49152, 1), (2, 20001, 256), (8, 131075, 50), (5, 4097, 7),
                     (1, 600_003, 100)]:
        lg = rng.normal(0, 3, (B, Vv)).astype(np.float32)
        for r in range(B):
            lg[r, rng.choice(Vv, 6, replace=False)] = lg[r].max() + 0.5
        hists = [list(rng.integers(-2, Vv + 2, int(rng.integers(0, 400)))) + [int(np.argmax(lg[r]))]
                 for r in range(B)]
        h, off = csr(hists)
        p = V.params_array(n=1, temp=0.9, top_k=k, top_p=0.9, min_p=0.02, repeat=1.2, repeat_last=0, seed=9)
        log("topk split", dmode, B, Vv, k)
        run = Run(ctx, lg, p, h, off, cand_cap=64)
        run.report()
        assert (run.info["path"] == V.PATH_SMALLK).all()
    # the reference's own draw stream, shared parameters: each row's state advances once per pick
    B, Vv = 4, 151936
    lg = rng.normal(0, 3, (B, Vv)).astype(np.float32)
    p = V.params_array(n=1, temp=0.8, top_k=40, top_p=0.95, repeat=1.0, repeat_last=0, seed=9)
    st = np.zeros((B, 2), np.uint64)
    for r in range(B):
        s0 = O.rng_seed(1000 + r)
        st[r] = [s0[0], s0[1]]
    dst = torch.from_numpy(st.view(np.int64).copy()).cuda()
    d = torch.from_numpy(lg).cuda()
    pr = V.Params(*[p[0][f].item() for f in V.SAMPLING_DTYPE.names])
    for step in range(3):
        log("topk split xorshift", dmode, step)
        ids = ctx.pick_batch(d, pr, u_mode=V.U_XORSHIFT, rng_state=dst).cpu().numpy()
        u = np.zeros(B)
        for r in range(B):
            s1 = (O.ctypes.c_uint64 * 2)(int(st[r, 0]), int(st[r, 1]))
            u[r] = O.rng_unit(s1)
            st[r] = [s1[0], s1[1]]
        assert (ids == O.pick_rows(lg, p, u=u)[0]).all()
        assert (dst.cpu().numpy().view(np.uint64) == st).all()


@pytest.mark.parametrize("kind", ["topp", "minp", "topk", "capped", "capped_minp", "flat"])
def test_general_path_two_workgroups_per_cu(kind):
    """Shared-parameter batches of general rows without a penalty and with more rows than the device
    has CUs run on two 512-thread workgroups per CU (the wide workload's launch): top-p, min-p, a
    top-k restriction above 256, rows wider than the buckets' 64 temp (capped, with and without a
    min-p threshold small enough to keep the overflow bucket) and tied rows that the exact redo
    takes; every comparison of the parity bar against the oracle."""
    import torch

    ctx = mode_ctx("rows")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = np.random.default_rng({"topp": 91, "minp": 92, "topk": 93, "capped": 94, "capped_minp": 95, "flat": 96}[kind])
    B, Vv = cus + 37, 5003
    lg = rng.normal(0.0, 1.0, (B, Vv))
    prm = dict(temp=1.0, top_k=0, top_p=0.9, min_p=0.0, repeat=1.0, repeat_last=0, seed=int(rng.integers(1, 1 << 62)))
    if kind == "minp":
        lg[:, rng.integers(0, Vv, 8)] += 5.0
        prm.update(temp=0.7, top_p=0.95, min_p=0.05)
    elif kind == "topk":
        prm.update(top_k=1000, top_p=0.9)
    elif kind == "capped":
        lg = rng.normal(0.0, 40.0, (B, Vv))
        prm.update(temp=0.5, top_p=0.99)
    elif kind == "capped_minp":
        lg = rng.normal(0.0, 40.0, (B, Vv))
        prm.update(temp=0.5, top_p=0.99, min_p=1e-30)
    elif kind == "flat":
        Vv = 5004
        lg = np.zeros((B, Vv))
        prm.update(top_p=0.5)
    p = V.params_array(n=1, **prm)
    h, off = csr([list(rng.integers(0, Vv, 50)) for _ in range(B)])  # ignored: repeat 1
    log("two workgroups per CU", kind, B, Vv)
    run = Run(ctx, lg.astype(np.float32), p, h, off, cand_cap=128)
    run.report()
    assert (run.info["path"] == V.PATH_GENERAL).all()
    if kind == "flat":
        assert (run.info["flags"] & V.FLAG_SEQ_CUTS).all(), run.info["flags"]


def test_general_path_all_rows_marked(ctx):
    """Every row of a batch goes to the exact redo: 40 rows of 151,936 equal logits with top-p 0.5
    (the top-p sum meets top_p exactly at an even count), a third with a penalised history, on the
    redo's blocked sort and staged sums, in every slot at once; keep counts, ids and draw sets equal
    the oracle's, and every row carries VSMP_FLAG_SEQ_CUTS."""
    rng = np.random.default_rng(81)
    B, Vv = 40, 151936
    lg = np.zeros((B, Vv), np.float32)
    p = V.params_array(n=B, temp=1.0, top_k=0, top_p=0.5, min_p=0.0, repeat=1.0, repeat_last=0, seed=5)
    p["repeat"][::3] = 1.2
    p["seed"] = rng.integers(1, 1 << 62, B)
    h, off = csr([list(rng.integers(0, Vv, 300)) if r % 3 == 0 else [] for r in range(B)])
    log("all rows marked", B, Vv)
    run = Run(ctx, lg, p, h, off, cand_cap=128)
    run.report()
    assert (run.info["flags"] & V.FLAG_SEQ_CUTS).all(), run.info["flags"]
    assert (run.info["keep"] == run.o_info["keep"]).all() and (run.ids == run.o_ids).all()
