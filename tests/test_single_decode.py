"""The single-row decode workload (1 x 49152, seed 42, 64-id history) as the compiled reference ran
it: 10,000 consecutive draws on the same row (tests/golden/single_draws_golden.npz), replayed on
the GPU three ways, each equal to the reference's ids draw for draw:
- the drop-in verbo::Sampler (host row copied per pick, the draw stream on the host: the path
  verbo's generate takes);
- vsmp_pick_batch on the device-resident row with the reference's xorshift stream on the device
  (VSMP_U_XORSHIFT), one call per draw, every id kept on the device;
- the same calls captured into a HIP graph (100 per graph) and replayed 100 times.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle as O
import verbo_amd as V
from helpers import log, mode_ctx
from verbo_amd import workloads as W

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden" / "single_draws_golden.npz"


@pytest.fixture(scope="module")
def single():
    z = np.load(GOLD, allow_pickle=False)
    w = W.make("single")
    c = z["cfg"][0]
    return w, V.Params(*[c[f].item() for f in V.SAMPLING_DTYPE.names]), z["ids"]


def test_drop_in_sampler_10000_draws(single):
    w, p, gold = single
    log("drop-in sampler, 10000 draws")
    s = V.Sampler(p)
    for t in w.hist:
        s.accept(int(t))
    got = np.array([s.pick(w.logits[0]) for _ in range(gold.size)], np.int32)
    assert (got == gold).all(), int(np.argmax(got != gold))


def _device_state(p):
    import torch

    st = O.rng_seed(int(p.seed))
    return torch.from_numpy(np.array([st[0], st[1]], np.uint64).view(np.int64)).cuda()


def test_device_resident_10000_draws(single):
    import torch

    w, p, gold = single
    ctx = mode_ctx(None)
    d = torch.from_numpy(w.logits).cuda()
    h, ho = torch.from_numpy(w.hist).cuda(), torch.from_numpy(w.hist_off).cuda()
    rng = _device_state(p)
    out = torch.full((gold.size,), -1, dtype=torch.int32, device="cuda")
    log("device-resident, 10000 calls")
    for i in range(gold.size):
        ctx.pick_batch(d, p, h, ho, V.U_XORSHIFT, rng_state=rng, out=out[i:i + 1])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert (got == gold).all(), int(np.argmax(got != gold))


def test_graph_replayed_10000_draws(single):
    import torch

    w, p, gold = single
    ctx = mode_ctx(None)
    d = torch.from_numpy(w.logits).cuda()
    h, ho = torch.from_numpy(w.hist).cuda(), torch.from_numpy(w.hist_off).cuda()
    rng = _device_state(p)
    per = 100
    ring = torch.full((per,), -1, dtype=torch.int32, device="cuda")
    ctx.pick_batch(d, p, h, ho, V.U_XORSHIFT, rng_state=_device_state(p), out=ring[:1])  # sizes the scratch
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            for i in range(per):
                ctx.pick_batch(d, p, h, ho, V.U_XORSHIFT, rng_state=rng, out=ring[i:i + 1], stream=st)
    torch.cuda.synchronize()
    rng.copy_(_device_state(p))  # the capture ran nothing: start the stream afresh
    got = []
    log("graph replays", gold.size // per)
    for _ in range(gold.size // per):
        g.replay()
        torch.cuda.synchronize()
        got.append(ring.cpu().numpy().copy())
    got = np.concatenate(got)
    assert (got == gold).all(), int(np.argmax(got != gold))


def test_device_sampler_reset_after_queued_picks(single):
    """vsmp_dsampler_reset issued while picks are still queued on the caller's stream lands after
    them: the queued picks give the reference's first draws, and after the reset (and the history
    accepted again) the stream starts over with the same draws."""
    import ctypes

    import torch

    w, p, gold = single
    lib = V.load_library()
    P_ = ctypes.c_void_p
    lib.vsmp_dsampler_new.restype, lib.vsmp_dsampler_new.argtypes = P_, [ctypes.c_int, ctypes.POINTER(V.Params)]
    lib.vsmp_dsampler_free.argtypes = [P_]
    lib.vsmp_dsampler_reset.argtypes = [P_]
    lib.vsmp_dsampler_accept.argtypes = [P_, P_, ctypes.c_int, P_]
    lib.vsmp_dsampler_pick.argtypes = [P_, P_, ctypes.c_int, P_]
    lib.vsmp_dsampler_pick_async.argtypes = [P_, P_, ctypes.c_int, P_, P_]
    s = lib.vsmp_dsampler_new(0, ctypes.byref(p))
    assert s, V.load_library().vsmp_last_error()
    try:
        st = torch.cuda.Stream()
        sp = ctypes.c_void_p(st.cuda_stream)
        d = torch.from_numpy(w.logits[0]).cuda()
        hist = np.ascontiguousarray(w.hist, np.int32)
        n = 300
        out = torch.full((n,), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        log("device sampler: picks queued, then reset")
        assert lib.vsmp_dsampler_accept(s, hist.ctypes.data, hist.size, sp) == 0
        for i in range(n):
            assert lib.vsmp_dsampler_pick_async(s, d.data_ptr(), w.V, out[i:i + 1].data_ptr(), sp) == 0
        assert lib.vsmp_dsampler_reset(s) == 0  # nothing waited for the stream before this
        assert lib.vsmp_dsampler_accept(s, hist.ctypes.data, hist.size, sp) == 0
        again = [lib.vsmp_dsampler_pick(s, d.data_ptr(), w.V, sp) for _ in range(5)]
        st.synchronize()
        got = out.cpu().numpy()
        assert (got == gold[:n]).all(), int(np.argmax(got != gold[:n]))
        assert again == [int(x) for x in gold[:5]], (again, gold[:5])
    finally:
        lib.vsmp_dsampler_free(s)


def test_host_picks_interleaved_with_batched_picks():
    """Host-row picks return as soon as their id reaches host memory (greedy and small-k rows, no
    diagnostics); batched picks issued on another stream right after them, with the same context,
    run after them on the GPU. Rows of 151,936 logits, so the batched small-k and greedy picks take
    the split kernels, whose scratch the context shares; every id against the oracle."""
    import torch

    rng = np.random.default_rng(11)
    Vv = 151936
    ctx = V.Context(0)
    st = torch.cuda.Stream()
    cases = []
    for i in range(24):
        row = (rng.standard_normal(Vv) * 2.5).astype(np.float32)
        row[rng.integers(0, Vv, 6)] += 9.0
        hist = rng.integers(0, Vv, 48).astype(np.int32)
        temp = 0.0 if i % 3 == 0 else 0.8
        p = V.Params(temp=temp, top_k=40, top_p=0.9, min_p=0.05, repeat=1.2, repeat_last=32, seed=1)
        c = O.sampling(temp=temp, top_k=40, top_p=0.9, min_p=0.05, repeat=1.2, repeat_last=32, seed=1)
        u = float(rng.random())
        cases.append((row, hist, p, c, u, O.pick(row, c, hist, u)[0]))
    log("host picks interleaved with batched picks")
    out = torch.full((len(cases),), -1, dtype=torch.int32, device="cuda")
    got_host = []
    for i, (row, hist, p, c, u, want) in enumerate(cases):
        got_host.append(ctx.pick_host(row, p, hist, u))
        d = torch.from_numpy(row).cuda().view(1, Vv)
        h = torch.from_numpy(hist).cuda()
        ho = torch.tensor([0, hist.size], dtype=torch.int32, device="cuda")
        uu = torch.tensor([u], dtype=torch.float64, device="cuda")
        torch.cuda.current_stream().synchronize()  # the inputs' copies, not the host pick
        ctx.pick_batch(d, p, h, ho, V.U_SUPPLIED, u=uu, out=out[i:i + 1], stream=st)
    st.synchronize()
    want = [x[-1] for x in cases]
    assert got_host == want, (got_host, want)
    assert out.cpu().tolist() == want
