"""Randomised batches against the oracle: every comparison of the parity bar (tests/helpers.py) on
300 seeded cases that mix what the other tests take one at a time. Row widths from 777 to 151,936
logits; normal, spiky, coarse-valued (ties), wide and cold (values spread far beyond 64
temperatures) rows; shared and per-row parameters over greedy, top-k 40, top-k 300 and 1000 and
top-k off, top-p from 0.5 to 1, min-p down to 1e-30, repeat above and below 1 with histories that
hold out-of-range ids; the planner's mode, rows and slices; batches of 3 to 300 rows (300 unpenalised
general rows with shared parameters run as two 512-thread workgroups per CU).

The LM head's pick (vsmp_head_pick) takes its own sweep: random bf16 hidden states and heads of 64
to 896 hidden elements and 1,000 to 151,936 columns, batches of 1 to 257 rows on the route by batch
size or the fused route pinned, every sampling mode, checked against the oracle on the logits the
head itself produces.

VSMP_SWEEP_CASES / VSMP_SWEEP_SEED and VSMP_HEAD_SWEEP_CASES / VSMP_HEAD_SWEEP_SEED run longer
sweeps, or other seeds, of the same generators (defaults 300 / 2024 and 60 / 2025)."""
import os

import numpy as np
import pytest

import verbo_amd as V
from helpers import Run, csr, log, mode_ctx

pytestmark = pytest.mark.gpu

N_CASES = int(os.environ.get("VSMP_SWEEP_CASES", "300"))
SEED = int(os.environ.get("VSMP_SWEEP_SEED", "2024"))


def case(rng):
    Vv = int(rng.choice([777, 4099, 20000, 50257, 128256, 151936]))
    B = int(rng.choice([3, 17, 64, 300])) if Vv < 100000 else int(rng.choice([3, 17, 64]))
    kind = str(rng.choice(["normal", "spiky", "wide", "flat", "cold"]))
    sd = float(rng.choice([0.3, 1.0, 3.0]))
    lg = rng.normal(0, sd, (B, Vv))
    if kind == "spiky":
        for r in range(B):
            lg[r, rng.integers(0, Vv, 12)] += rng.uniform(3, 10, 12)
    elif kind == "flat":
        lg[:] = np.round(lg * 4) / 4
    elif kind == "cold":
        lg *= 20.0

    def one():
        return dict(temp=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])),
                    top_k=int(rng.choice([0, 0, 0, 40, 300, 1000])),
                    top_p=float(rng.choice([1.0, 0.5, 0.9, 0.95, 0.99])),
                    min_p=float(rng.choice([0.0, 0.0, 0.01, 0.05, 1e-30])),
                    repeat=float(rng.choice([1.0, 1.0, 1.1, 1.3, 0.8])), repeat_last=int(rng.choice([0, 64])),
                    seed=int(rng.integers(1, 1 << 62)))

    per_row = bool(rng.random() < 0.5)
    p = V.params_array([one() for _ in range(B)]) if per_row else V.params_array(n=1, **one())
    h, off = csr([list(rng.integers(-2, Vv + 2, int(rng.integers(0, 600)))) for _ in range(B)])
    mode = rng.choice([None, "rows", "slices"])
    return dict(kind=kind, sd=sd, B=B, V=Vv, per_row=per_row, mode=None if mode is None else str(mode)), lg, p, h, off


def test_randomised_batches():
    rng = np.random.default_rng(SEED)
    near = 0
    for i in range(N_CASES):
        desc, lg, p, h, off = case(rng)
        log("sweep case", i, desc)
        run = Run(mode_ctx(desc["mode"]), lg.astype(np.float32), p, h, off, cand_cap=64)
        nd, nm = run.report()
        assert nm == 0, (i, desc, nd, nm)
        near += nd
    log("sweep:", N_CASES, "cases,", near, "draws within 1e-6 of a CDF boundary, none of them mismatched")


N_HEAD_CASES = int(os.environ.get("VSMP_HEAD_SWEEP_CASES", "60"))
HEAD_SEED = int(os.environ.get("VSMP_HEAD_SWEEP_SEED", "2025"))


def head_case(rng):
    import torch

    B = int(rng.choice([1, 5, 16, 33, 64, 100, 257]))
    Vv = int(rng.choice([1000, 4095, 4097, 9000, 32000, 151936]))
    if Vv > 100000:
        B = min(B, 64)
    D = int(rng.choice([64, 128, 256, 896]))
    x = rng.standard_normal((B, D)).astype(np.float32)
    w = (rng.standard_normal((Vv, D)) * (3.0 / np.sqrt(D))).astype(np.float32)
    w[rng.integers(0, Vv, 8)] *= 3.0
    hidden = torch.from_numpy(x).to(torch.bfloat16).cuda()
    head = torch.from_numpy(w).to(torch.bfloat16).cuda()

    def one():
        return dict(temp=float(rng.choice([0.0, 0.5, 0.8, 1.2])), top_k=int(rng.choice([0, 1, 40, 256, 300])),
                    top_p=float(rng.choice([1.0, 0.9, 0.95])), min_p=float(rng.choice([0.0, 0.05])),
                    repeat=float(rng.choice([1.0, 1.1, 0.8])), repeat_last=int(rng.choice([0, 64])),
                    seed=int(rng.integers(1, 1 << 62)))

    per_row = bool(rng.random() < 0.4) and B > 1
    p = V.params_array([one() for _ in range(B)]) if per_row else V.params_array(n=1, **one())
    h, off = csr([list(rng.integers(-2, Vv + 2, int(rng.integers(0, 300)))) for _ in range(B)])
    route = rng.choice(["auto", "fused"])
    return dict(B=B, V=Vv, D=D, per_row=per_row, route=str(route)), hidden, head, p, h, off


def test_randomised_head_batches():
    import torch

    rng = np.random.default_rng(HEAD_SEED)
    near = 0
    for i in range(N_HEAD_CASES):
        desc, hidden, head, p, h, off = head_case(rng)
        log("head sweep case", i, desc)
        ctx = mode_ctx(None, None if desc["route"] == "auto" else "fused")
        logits = ctx.head_logits(hidden, head)
        torch.cuda.synchronize()

        def pick(pr, dh, dho, du, **dbg):
            return ctx.head_pick(hidden, head, pr, dh, dho, V.U_SUPPLIED, du, **dbg)

        run = Run(ctx, logits.cpu().numpy(), p, h, off, cand_cap=64, pick=pick)
        nd, nm = run.report()
        assert nm == 0, (i, desc, nd, nm)
        near += nd
    log("head sweep:", N_HEAD_CASES, "cases,", near, "draws within 1e-6 of a CDF boundary, none of them mismatched")
