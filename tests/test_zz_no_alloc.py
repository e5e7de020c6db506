"""vsmp_pick_batch_noalloc, the entry point that allocates nothing (its scratch is one static
device array per GPU), against vsmp_pick_batch in row mode (the same kernels with the context's
scratch) on the same inputs: two calls in a row, the second with a smaller batch, each with
every diagnostic. Ids, keep counts, last ids, penalised-index bitmaps and candidate lists are
bit-exact; the fp64 sums agree within 1e-12 (the general path's LDS atomics add in any order).
The batches hold greedy, small-k and general rows, and rows of tied logits whose top-p cut lies at
rounding distance, which the exact redo takes in its one sort slot. Calls beyond the limits fail
with an error before any GPU work."""
import numpy as np
import pytest

import verbo_amd as V
from helpers import csr, log, mode_ctx

pytestmark = pytest.mark.gpu


def _mixed_batch(rng, B, Vv, n_tied):
    lg = rng.normal(0, 2.0, (B, Vv)).astype(np.float32)
    p = np.zeros(B, V.SAMPLING_DTYPE)
    p["temp"] = rng.choice([0.0, 0.6, 1.0], B)
    p["top_k"] = rng.choice([0, 0, 40, 300], B)
    p["top_p"] = rng.choice([0.9, 0.95, 1.0], B)
    p["min_p"] = rng.choice([0.0, 0.05], B)
    p["repeat"] = rng.choice([1.0, 1.2], B)
    p["repeat_last"] = 0
    p["seed"] = rng.integers(1, 1 << 62, B)
    for r in range(n_tied):  # all logits equal, top-p 0.5 of an even V: the cut meets top_p exactly
        lg[r] = 0.0
        p["temp"][r], p["top_k"][r], p["top_p"][r], p["min_p"][r] = 1.0, 0, 0.5, 0.0
    h, off = csr([rng.integers(0, Vv, int(rng.integers(0, 400))) for _ in range(B)])
    return lg, p, h, off, rng.random(B)


def _run(fn, lg, p, h, off, u, per_row=True):
    import torch

    B, Vv = lg.shape
    d = torch.from_numpy(lg).cuda()
    prm = V.to_device_params(p) if per_row else V.Params(*[p[0][f].item() for f in V.SAMPLING_DTYPE.names])
    info = torch.zeros(B * 72, dtype=torch.uint8, device="cuda")
    cid = torch.full((B, 64), -1, dtype=torch.int32, device="cuda")
    cpr = torch.zeros((B, 64), dtype=torch.float64, device="cuda")
    pen = torch.full((B, (Vv + 31) // 32), -1, dtype=torch.int32, device="cuda")
    out = fn(d, prm, torch.from_numpy(h).cuda(), torch.from_numpy(off).cuda(), V.U_SUPPLIED, torch.from_numpy(u).cuda(),
             info=info, cand_ids=cid, cand_pr=cpr, pen_bits=pen)
    torch.cuda.synchronize()
    return out.cpu().numpy(), V.row_info(info), cid.cpu().numpy(), cpr.cpu().numpy(), pen.cpu().numpy()


def _same(a, b):
    ids_a, inf_a, c_a, p_a, pen_a = a
    ids_b, inf_b, c_b, p_b, pen_b = b
    assert (ids_a == ids_b).all()
    for f in ("id", "path", "k", "keep_minp", "keep", "rank", "last_id", "flags", "n_pen"):
        assert (inf_a[f] == inf_b[f]).all(), f
    assert (inf_a["mx"] == inf_b["mx"]).all()
    for f in ("sum", "tot"):
        assert np.allclose(inf_a[f], inf_b[f], rtol=1e-12, atol=0), f
    assert (c_a == c_b).all()
    assert np.allclose(p_a, p_b, rtol=1e-12, atol=0)
    assert (pen_a == pen_b).all()


def test_noalloc_equals_the_batched_entry_point():
    ctx = mode_ctx("rows")
    rng = np.random.default_rng(71)
    for B, Vv, n_tied in ((96, 151936, 3), (24, 49152, 2)):  # the second call is smaller
        lg, p, h, off, u = _mixed_batch(rng, B, Vv, n_tied)
        log("no-alloc per-row", B, Vv)
        want = _run(ctx.pick_batch, lg, p, h, off, u)
        got = _run(V.pick_batch_noalloc, lg, p, h, off, u)
        _same(got, want)
        tied = want[1]["flags"][:n_tied]
        assert (tied & V.FLAG_SEQ_CUTS).all(), tied  # the exact redo ran on the tied rows
    # shared parameters: a general batch with a top-p cut, then a smaller small-k batch
    for B, Vv, shared in ((40, 131072, dict(temp=1.0, top_k=0, top_p=0.5)),
                          (8, 20000, dict(temp=0.8, top_k=50, top_p=0.95, min_p=0.05))):
        lg, p, h, off, u = _mixed_batch(rng, B, Vv, 2 if shared["top_k"] == 0 else 0)
        p1 = V.params_array(n=1, repeat=1.1, repeat_last=0, seed=5, **shared)
        log("no-alloc shared", B, Vv, shared)
        _same(_run(V.pick_batch_noalloc, lg, p1, h, off, u, per_row=False),
              _run(ctx.pick_batch, lg, p1, h, off, u, per_row=False))


def test_noalloc_rejects_sizes_beyond_its_scratch():
    import torch

    p = V.Params()
    with pytest.raises(V.VsmpError, match="at most 2048 rows of at most 262144"):
        V.pick_batch_noalloc(torch.zeros((1, 262148), device="cuda"), p)
    with pytest.raises(V.VsmpError, match="at most 2048 rows"):
        V.pick_batch_noalloc(torch.zeros((2049, 8), device="cuda"), p)
