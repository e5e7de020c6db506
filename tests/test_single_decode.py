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
