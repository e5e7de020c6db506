"""The LM head on the GPU and the pick fused into it (vsmp_head_logits, vsmp_head_pick).

The head's product (reference src/session.cpp:169, matmul(m->head, ...)) is checked against a
plain fp32 product of the same bf16 operands on the CPU. vsmp_head_pick is checked, on its route
by batch size and with the fused route pinned for every batch, against the oracle (the reference's
Sampler::pick, src/sampler.cpp:50-109) on the logits the head itself produces, with every
comparison rule of the batched path (penalised ids, keep counts, candidate ids, sums, ids), and
against vsmp_pick_batch on those logits, field for field.
"""
import numpy as np
import pytest

import verbo_amd as V
from helpers import Run, csr, log, mode_ctx

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "fused"])
def ctx(request):
    """vsmp_head_pick's route by batch size (fused for 16 to 64 rows, the head's logits written and
    the batched pick otherwise), and the fused route pinned for every batch."""
    import torch

    assert torch.cuda.is_available(), "the gpu tests need a ROCm device"
    return mode_ctx(None, None if request.param == "auto" else request.param)


def bf16(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def operands(seed, B, Vv, D, spread=3.0):
    """Random bf16 hidden [B, D] and head [V, D] (device) whose logits have about `spread` standard
    deviation, plus a few strong columns so that rows have clear leaders."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, D)).astype(np.float32)
    w = (rng.standard_normal((Vv, D)) * (spread / np.sqrt(D))).astype(np.float32)
    hot = rng.choice(Vv, size=min(40, Vv), replace=False)
    w[hot] += (rng.standard_normal((len(hot), D)) * (2.0 / np.sqrt(D))).astype(np.float32)
    return bf16(x).cuda(), bf16(w).cuda()


def fp32_reference(hidden, head):
    """hidden @ head.T in fp32 on the CPU, and the bound |hidden| @ |head|.T of its rounding."""
    import torch

    x = hidden.float().cpu()
    w = head.float().cpu()
    return (x @ w.T).numpy(), (x.abs() @ w.abs().T).numpy()


@pytest.mark.parametrize("B,Vv,D", [(1, 1000, 64), (37, 4099, 128), (130, 5000, 192), (64, 8269, 256),
                                    (256, 20000, 896), (8, 5000, 4096), (200, 151936, 896)])
def test_head_logits_match_fp32_product(ctx, B, Vv, D):
    """Every logit within 2e-5 of sum |x_d w_d| of the fp32 product: the fp32 accumulation of D
    exact bf16 products in another order (and one that swaps rows or columns is off by far more)."""
    import torch

    log("head logits", B, Vv, D)
    hidden, head = operands(11 + B, B, Vv, D)
    got = ctx.head_logits(hidden, head)
    torch.cuda.synchronize()
    want, mag = fp32_reference(hidden, head)
    g = got.cpu().numpy()
    err = np.abs(g - want)
    assert (err <= 2e-5 * mag + 1e-30).all(), float(np.max(err / np.maximum(mag, 1e-30)))


@pytest.mark.parametrize("Vv,D", [(12345, 320), (12345, 896), (151936, 896)])
def test_head_logits_do_not_depend_on_the_batch(ctx, Vv, D):
    """A row's logits are the same bits whether it is computed alone, in a batch of 77 or of 256
    (different tile shapes; at 151,936 columns the 256-row batch's product is two launches, the
    columns of the whole rounds on 256 x 256 tiles and the rest on 256 x 128 tiles), and whether
    vsmp_head_pick writes them or vsmp_head_logits does."""
    import torch

    log("head logits across tiles", Vv, D)
    hidden, head = operands(5, 256, Vv, D)
    full = ctx.head_logits(hidden, head)
    mid = ctx.head_logits(hidden[:77].contiguous(), head)
    one = ctx.head_logits(hidden[200:201].contiguous(), head)
    ldl = (Vv + 3) // 4 * 4
    lg = torch.full((256, ldl), float("nan"), dtype=torch.float32, device="cuda")
    ctx.head_pick(hidden, head, V.Params(temp=0.8, top_k=50, top_p=0.95, repeat=1.0), logits=lg)
    torch.cuda.synchronize()
    f = full.cpu().numpy()
    assert np.array_equal(mid.cpu().numpy(), f[:77])
    assert np.array_equal(one.cpu().numpy(), f[200:201])
    assert np.array_equal(lg[:, :Vv].cpu().numpy(), f)


def head_run(ctx, hidden, head, params, hist=None, hist_off=None, cand_cap=128):
    """The fused pick through Run: the oracle and Run's comparisons on the head's own logits."""
    import torch

    logits = ctx.head_logits(hidden, head)
    torch.cuda.synchronize()

    def pick(pr, dh, dho, du, **dbg):
        return ctx.head_pick(hidden, head, pr, dh, dho, V.U_SUPPLIED, du, **dbg)

    return Run(ctx, logits.cpu().numpy(), params, hist, hist_off, cand_cap=cand_cap, pick=pick)


def same_as_pick_batch(ctx, r, hist, hist_off):
    """The head pick's ids and row diagnostics equal vsmp_pick_batch's on the same logits: the
    general path's fp64 sums (top-k off or above 256) to 1e-12, every other field, and every field
    of greedy and small-k rows, to the bit."""
    b = Run(ctx, r.logits, r.params, hist, hist_off, u=r.u, cand_cap=r.cand_cap)
    assert np.array_equal(r.ids, b.ids)
    for f in ("id", "path", "k", "keep_minp", "keep", "rank", "last_id", "n_pen", "mx", "u"):
        assert np.array_equal(r.info[f], b.info[f]), f
    gen = r.info["path"] == 2
    for f in ("sum", "tot"):
        assert np.array_equal(r.info[f][~gen], b.info[f][~gen]), f
        assert np.allclose(r.info[f][gen], b.info[f][gen], rtol=1e-12, atol=0), f
    assert np.array_equal(r.cand, b.cand)
    assert all(np.array_equal(x, y) for x, y in zip(r.pen, b.pen))


PARAM_SETS = {
    # the peaked bench's sampler: top-k 50, top-p .95, min-p .05, repeat 1.1 over 64 of 512 ids
    "topk50": dict(temp=0.8, top_k=50, top_p=0.95, min_p=0.05, repeat=1.1, repeat_last=64),
    "greedy": dict(temp=0.0, top_k=40, top_p=0.9, repeat=1.3, repeat_last=0),
    "topk1": dict(temp=0.7, top_k=1, top_p=0.9, repeat=1.0),
    "topk256": dict(temp=1.3, top_k=256, top_p=0.9, min_p=0.0, repeat=1.05, repeat_last=128),
    # repeat < 1 raises a history logit: the bound on raw logits is lowered for it
    "raise": dict(temp=0.6, top_k=40, top_p=0.99, min_p=0.01, repeat=0.7, repeat_last=0),
    "general": dict(temp=0.9, top_k=0, top_p=0.9, repeat=1.1, repeat_last=64),
}


@pytest.mark.parametrize("name", sorted(PARAM_SETS))
@pytest.mark.parametrize("B,Vv,D", [(256, 151936, 896), (33, 20000, 128), (5, 4100, 64), (3, 1000, 64)])
def test_head_pick_matches_oracle(ctx, name, B, Vv, D):
    """Shared parameters, histories that hit the probe columns and the rest (out-of-range ids too):
    the fused pick equals the oracle's on the head's logits, and vsmp_pick_batch's."""
    log("head pick", name, B, Vv, D)
    rng = np.random.default_rng(sum(map(ord, name)) * 1000 + B)
    hidden, head = operands(7 + B, B, Vv, D)
    hists = []
    for r in range(B):
        n = int(rng.integers(0, 513))
        h = rng.integers(0, Vv, n)
        h[: n // 4] = rng.integers(0, min(Vv, 4096), n // 4)  # in the probe columns
        if n > 3:
            h[1] = Vv + 5
            h[2] = -3
        hists.append(h)
    hist, off = csr(hists)
    params = V.params_array(n=1, seed=99, **PARAM_SETS[name])
    r = head_run(ctx, hidden, head, params, hist, off)
    near, mism = r.report()
    log("  counts", r.counts)
    assert mism == 0
    same_as_pick_batch(ctx, r, hist, off)


def test_head_pick_per_row_parameters(ctx):
    """Per-row parameters mixing greedy, small-k and general rows (the general rows' logits written
    and sampled by the general path), with per-row histories."""
    B, Vv, D = 96, 32000, 256
    rng = np.random.default_rng(3)
    hidden, head = operands(21, B, Vv, D)
    rows = []
    for r in range(B):
        kind = r % 4
        if kind == 0:
            rows.append(dict(temp=0.0, repeat=1.2, repeat_last=32, seed=r))
        elif kind == 1:
            rows.append(dict(temp=0.8, top_k=int(rng.integers(1, 257)), top_p=0.9, min_p=0.02, repeat=1.1, seed=r))
        elif kind == 2:
            rows.append(dict(temp=1.1, top_k=0, top_p=0.8, min_p=0.05, repeat=1.0, seed=r))
        else:
            rows.append(dict(temp=0.5, top_k=40, top_p=1.0, repeat=0.9, repeat_last=16, seed=r))
    params = V.params_array(rows)
    hist, off = csr([rng.integers(0, Vv, int(rng.integers(0, 100))) for _ in range(B)])
    r = head_run(ctx, hidden, head, params, hist, off)
    near, mism = r.report()
    log("  counts", r.counts)
    assert mism == 0
    same_as_pick_batch(ctx, r, hist, off)


def onehot_head(values):
    """hidden = one-hot rows and head columns = `values` (bf16-exact): the head's logits are exactly
    values[r] for row r (one nonzero product per logit)."""
    B, Vv = values.shape
    D = 64
    hidden = np.zeros((B, D), np.float32)
    head = np.zeros((Vv, D), np.float32)
    for r in range(B):
        hidden[r, r % D] = 1.0
        head[:, r % D] = values[r]
    return bf16(hidden).cuda(), bf16(head).cuda()


def test_head_pick_ties_and_flat_rows(ctx):
    """Rows whose logits tie: all equal (every column a candidate: the finish takes them in several
    rounds), a few values repeated across the row (ties at the bound and at the top), and a zero
    row with a penalised history; greedy and small-k parameters."""
    rng = np.random.default_rng(8)
    Vv = 20000
    vals = np.zeros((6, Vv), np.float32)
    vals[1] = rng.choice(np.array([1.0, 2.0, 3.0, 3.5], np.float32), Vv)
    vals[2] = np.float32(-1.5)
    vals[3] = rng.choice(np.array([0.0, 0.25, 0.5], np.float32), Vv)
    vals[3, rng.choice(Vv, 60, replace=False)] = 4.0
    vals[4, :] = 2.0
    vals[4, 5000:] = 2.5
    vals[5] = rng.integers(-8, 8, Vv).astype(np.float32) / 4
    hidden, head = onehot_head(vals)
    hist, off = csr([[0, 1, 2, 3, 3, 19999], [], [7, 8], [], list(range(4990, 5040)), [11] * 5])
    for p in (dict(temp=0.0, repeat=1.5, repeat_last=0), dict(temp=0.9, top_k=60, top_p=0.7, repeat=1.5, repeat_last=0),
              dict(temp=0.9, top_k=7, top_p=0.95, repeat=0.5, repeat_last=0)):
        log("ties", p)
        r = head_run(ctx, hidden, head, V.params_array(n=1, seed=4, **p), hist, off)
        near, mism = r.report()
        assert mism == 0
        same_as_pick_batch(ctx, r, hist, off)


def test_head_bad_arguments(ctx):
    import torch

    hidden, head = operands(1, 4, 1000, 64)
    with pytest.raises(V.VsmpError, match="multiple of 64"):
        ctx.head_logits(hidden[:, :32].contiguous(), head[:, :32].contiguous())
    big = torch.zeros((1, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(V.VsmpError, match="at most"):
        ctx.head_logits(big, torch.zeros(((1 << 19) + 1, 64), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(V.VsmpError, match="same number of columns"):
        ctx.head_logits(hidden, head[:, :32].contiguous())
    with pytest.raises(V.VsmpError, match="ldl"):
        ctx.head_pick(hidden, head, V.Params(), logits=torch.zeros((4, 999), device="cuda"))


def test_head_pick_row_tiles_padding_and_draw_modes(ctx):
    """300 rows (two row tiles of the main product, five of the probe), padded leading dimensions,
    and the device draw modes: with xorshift draws (the reference's stream, advanced in place) and
    with counter draws, the fused pick equals vsmp_pick_batch on the head's logits, and the streams
    end in the same state."""
    import torch

    B, Vv, D = 300, 9000, 192
    hidden_w, head_w = operands(31, B, Vv, D + 64)
    hidden = hidden_w[:, :D]  # row stride D + 64
    head = head_w[:, :D]
    logits = ctx.head_logits(hidden, head)
    rng = np.random.default_rng(12)
    hist, off = csr([rng.integers(0, Vv, int(rng.integers(0, 80))) for _ in range(B)])
    dh, dho = torch.from_numpy(hist).cuda(), torch.from_numpy(off).cuda()
    for p in (dict(temp=0.9, top_k=40, top_p=0.9, min_p=0.02, repeat=1.15, repeat_last=32, seed=8),
              dict(temp=0.0, repeat=1.2, repeat_last=16, seed=8)):
        prm = V.Params(*[V.params_array(n=1, **p)[0][f].item() for f in V.SAMPLING_DTYPE.names])
        state = torch.from_numpy(rng.integers(1, 1 << 62, 2 * B).astype(np.int64)).cuda()
        s1, s2 = state.clone(), state.clone()
        a = ctx.head_pick(hidden, head, prm, dh, dho, V.U_XORSHIFT, rng_state=s1)
        b = ctx.pick_batch(logits, prm, dh, dho, V.U_XORSHIFT, rng_state=s2)
        torch.cuda.synchronize()
        assert np.array_equal(a.cpu().numpy(), b.cpu().numpy()), p
        assert np.array_equal(s1.cpu().numpy(), s2.cpu().numpy()), p
    per_row = V.to_device_params(V.params_array(
        [dict(temp=0.7 + 0.001 * r, top_k=[0, 20, 300, 1][r % 4], top_p=0.9, repeat=1.1, seed=r) for r in range(B)]))
    a = ctx.head_pick(hidden, head, per_row, dh, dho, V.U_COUNTER, counter=5)
    b = ctx.pick_batch(logits, per_row, dh, dho, V.U_COUNTER, counter=5)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_head_pick_routes_agree():
    """VSMP_HEAD_ROUTE pins vsmp_head_pick's route. At 32 rows (fused by batch size) the whole route
    (the head's logits written, then the batched pick) and the fused one give the same ids, the
    same row diagnostics and the same candidate ids, for greedy, small-k and general parameters
    with penalised histories and counter draws."""
    import torch

    B, Vv, D = 32, 20000, 128
    hidden, head = operands(41, B, Vv, D)
    rng = np.random.default_rng(41)
    h, off = csr([list(rng.integers(0, Vv, 200)) for _ in range(B)])
    hist = torch.from_numpy(h).cuda()
    hoff = torch.from_numpy(off).cuda()
    for prm in (V.Params(temp=0.0, repeat=1.2, repeat_last=0), V.Params(temp=0.8, top_k=50, top_p=0.95,
                min_p=0.05, repeat=1.1, repeat_last=0, seed=5), V.Params(temp=1.0, top_k=0, top_p=0.9, repeat=1.1,
                repeat_last=64, seed=6)):
        got = {}
        for route in ("fused", "whole"):
            c = mode_ctx(None, route)
            info = torch.zeros(B * 72, dtype=torch.uint8, device="cuda")
            cand = torch.full((B, 64), -1, dtype=torch.int32, device="cuda")
            out = c.head_pick(hidden, head, prm, hist, hoff, V.U_COUNTER, counter=3, info=info, cand_ids=cand)
            torch.cuda.synchronize()
            got[route] = (out.cpu().numpy(), V.row_info(info), cand.cpu().numpy())
        (fo, fi, fc), (wo, wi, wc) = got["fused"], got["whole"]
        assert np.array_equal(fo, wo), prm
        for f in ("id", "path", "k", "keep_minp", "keep", "rank", "last_id", "n_pen", "mx", "u"):
            assert np.array_equal(fi[f], wi[f]), (prm, f)
        assert np.allclose(fi["sum"], wi["sum"], rtol=1e-12, atol=0) and np.allclose(fi["tot"], wi["tot"], rtol=1e-12, atol=0)
        assert np.array_equal(fc, wc), prm
