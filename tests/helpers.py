"""Shared test helpers: run the HIP sampler through the C ABI and the oracle on the same inputs,
then compare with the reference's tolerance rules.

Comparison rules (the parity bar), applied to every row:
- greedy ids, the penalised-index set (the kernels' own bitmaps), the largest penalised logit, k,
  the min-p and top-p keep counts, the draw set's last id and its first cand_cap ids in sorted
  order: bit-exact. The only exemption: a row the kernel itself flags as a min-p or top-p decision
  at rounding distance (VSMP_FLAG_MINP_NEAR / VSMP_FLAG_TOPP_NEAR) without having redone it in
  the reference's sequential order (VSMP_FLAG_SEQ_CUTS), where the oracle's margin is also below
  rounding distance (|acc - top_p| < 1e-11, |pr - thr| / thr < 1e-13); such rows are counted.
- probabilities (fp64 numerators, sums): within 1e-5 relative;
- sampled ids: equal, except where the draw lies within 1e-6 (relative) of a CDF boundary, or on
  an exempt row; those are counted, and the tests require the mismatches among them to be zero.
"""
import os
import sys

import numpy as np

import oracle as O
import verbo_amd as V

NEAR_TOPP = 1e-11
NEAR_MINP = 1e-13
NEAR_DRAW = 1e-6
PROB_RTOL = 1e-5


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


_CTX = {}


def mode_ctx(mode=None, head_route=None):
    """A context created under VSMP_MODE=mode (None: the planner's choice) and
    VSMP_HEAD_ROUTE=head_route (None: vsmp_head_pick's route by batch size), cached per pair: the
    library reads its tuning switches once, when a context is created."""
    key = (mode, head_route)
    if key not in _CTX:
        saved = {k: os.environ.pop(k, None) for k in ("VSMP_MODE", "VSMP_HEAD_ROUTE")}
        try:
            if mode:
                os.environ["VSMP_MODE"] = mode
            if head_route:
                os.environ["VSMP_HEAD_ROUTE"] = head_route
            _CTX[key] = V.Context(0)
        finally:
            for k, v in saved.items():
                os.environ.pop(k, None)
                if v is not None:
                    os.environ[k] = v
    return _CTX[key]


def csr(hists):
    off = np.zeros(len(hists) + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    flat = np.concatenate([np.asarray(h, np.int32) for h in hists]) if off[-1] else np.zeros(0, np.int32)
    return flat.astype(np.int32), off


class Run:
    """One batched GPU pick and the oracle's answer on the same inputs."""

    def __init__(self, ctx, logits, params, hist=None, hist_off=None, u=None, cand_cap=128, ld=None, device="cuda",
                 pick=None):
        """pick: None (ctx.pick_batch on the logits, uploaded), or a callable taking pick_batch's
        arguments (params, hist, hist_off, u and the diagnostic tensors as keywords) that makes the
        same pick some other way (the LM-head path, whose `logits` are the head's own output)."""
        import torch

        self.logits = np.ascontiguousarray(logits, np.float32)
        B, Vv = self.logits.shape
        self.B, self.V = B, Vv
        self.params = np.ascontiguousarray(params, dtype=V.SAMPLING_DTYPE)
        per_row = self.params.size == B and B > 1
        if u is None:
            u = np.array([O.counter_u(int(self.params[r if per_row else 0]["seed"]), r) for r in range(B)])
        self.u = np.asarray(u, np.float64)
        ld = ld or ((Vv + 3) // 4 * 4)
        buf = torch.zeros((B, ld), dtype=torch.float32)
        buf[:, :Vv] = torch.from_numpy(self.logits)
        dl = buf.to(device)[:, :Vv]
        dh = dho = None
        if hist is not None:
            dh = torch.from_numpy(np.ascontiguousarray(hist, np.int32) if len(hist) else np.zeros(1, np.int32)).to(device)
            dho = torch.from_numpy(np.ascontiguousarray(hist_off, np.int32)).to(device)
        du = torch.from_numpy(self.u).to(device)
        info = torch.zeros(B * 72, dtype=torch.uint8, device=device)
        cid = cpr = None
        if cand_cap:
            cid = torch.full((B, cand_cap), -1, dtype=torch.int32, device=device)
            cpr = torch.zeros((B, cand_cap), dtype=torch.float64, device=device)
        # garbage in the bitmaps: the call must write them whole
        pen = torch.full((B, (Vv + 31) // 32), -1, dtype=torch.int32, device=device)
        pr = V.Params(*[self.params[0][f].item() for f in V.SAMPLING_DTYPE.names]) if not per_row else \
            V.to_device_params(self.params, device)
        if pick is None:
            out = ctx.pick_batch(_rows_view(dl), pr, dh, dho, V.U_SUPPLIED, du, info=info, cand_ids=cid, cand_pr=cpr,
                                 pen_bits=pen)
        else:
            out = pick(pr, dh, dho, du, info=info, cand_ids=cid, cand_pr=cpr, pen_bits=pen)
        torch.cuda.synchronize()
        self.ids = out.cpu().numpy()
        self.info = V.row_info(info)
        self.cand = cid.cpu().numpy() if cid is not None else None
        self.cand_pr = cpr.cpu().numpy() if cpr is not None else None
        self.cand_cap = cand_cap
        self.pen = V.pen_ids(pen.cpu().numpy(), Vv)
        hmax = int(np.max(np.diff(hist_off))) if hist_off is not None and len(hist_off) > 1 else 0
        (self.o_ids, self.o_info, self.o_cand, self.o_pr,
         self.o_pen) = O.pick_rows(self.logits, self.params, hist, hist_off, self.u, cand_cap=cand_cap,
                                   pen_cap=max(hmax, 1))
        self.counts = {}

    def report(self):
        """Checks every row; returns (n_near_draw, n_mismatch_near) and raises on any other
        difference. self.counts: rows per category (near draws, exempt rows, sequential redos)."""
        gi, oi = self.info, self.o_info
        problems = []
        near = exempt = seq = near_mismatch = 0
        for r in range(self.B):
            o = oi[r]
            g = gi[r]
            gf = int(g["flags"])
            if not np.array_equal(self.pen[r], self.o_pen[r]):
                problems.append(f"row {r}: penalised ids differ ({len(self.pen[r])} vs {len(self.o_pen[r])})")
            if g["n_pen"] != o["n_pen"]:
                problems.append(f"row {r}: n_pen {g['n_pen']} != {o['n_pen']}")
            if g["id"] != self.ids[r]:
                problems.append(f"row {r}: out {self.ids[r]} != info.id {g['id']}")
            if gf & V.FLAG_CUTS_DIFFER:
                problems.append(f"row {r}: parallel and sequential cuts differ")
            if not np.float32(g["mx"]) == np.float32(o["mx"]):
                problems.append(f"row {r}: mx {g['mx']} != {o['mx']}")
            if o["greedy"]:
                if self.ids[r] != self.o_ids[r]:
                    problems.append(f"row {r}: greedy id {self.ids[r]} != oracle {self.o_ids[r]}")
                continue
            near_o = o["topp_margin"] < NEAR_TOPP or o["minp_margin"] < NEAR_MINP
            flagged = gf & (V.FLAG_TOPP_NEAR | V.FLAG_MINP_NEAR)
            redone = gf & V.FLAG_SEQ_CUTS
            set_amb = bool(near_o and flagged and not redone)
            exempt += int(set_amb)
            seq += int(bool(redone))
            draw_amb = o["draw_margin"] < NEAR_DRAW
            near += int(draw_amb)
            if g["k"] != o["k"]:
                problems.append(f"row {r}: k {g['k']} != {o['k']}")
            if not set_amb:
                if g["keep_minp"] != o["keep_minp"] or g["keep"] != o["keep"]:
                    problems.append(f"row {r}: keep ({g['keep_minp']},{g['keep']}) != ({o['keep_minp']},{o['keep']})")
                if g["last_id"] != o["last_id"]:
                    problems.append(f"row {r}: last id of the draw set {g['last_id']} != {o['last_id']}")
                if abs(g["tot"] - o["tot"]) > PROB_RTOL * abs(o["tot"]):
                    problems.append(f"row {r}: tot {g['tot']} vs {o['tot']}")
            if abs(g["sum"] - o["sum"]) > PROB_RTOL * abs(o["sum"]):
                problems.append(f"row {r}: sum {g['sum']} vs {o['sum']}")
            if self.ids[r] != self.o_ids[r]:
                if draw_amb or set_amb:
                    near_mismatch += 1
                else:
                    problems.append(f"row {r}: id {self.ids[r]} != oracle {self.o_ids[r]} "
                                    f"(draw margin {o['draw_margin']:.3g}, keep {o['keep']}, path {g['path']})")
            if self.cand is not None and not set_amb:
                m = min(int(o["keep"]), self.cand_cap)
                if not (self.cand[r, :m] == self.o_cand[r, :m]).all():
                    bad = int(np.argmax(self.cand[r, :m] != self.o_cand[r, :m]))
                    problems.append(f"row {r}: candidate ids differ from position {bad} of {m} (path {g['path']})")
                if self.cand_cap > m and (self.cand[r, m:] != -1).any():
                    problems.append(f"row {r}: candidate ids written past min(keep, cand_cap)")
                p, q = self.cand_pr[r, :m], self.o_pr[r, :m]
                if (np.abs(p - q) > PROB_RTOL * np.abs(q)).any():
                    problems.append(f"row {r}: candidate probabilities differ by {np.max(np.abs(p - q) / q):.3g}")
        if problems:
            raise AssertionError(f"{len(problems)} problems:\n" + "\n".join(problems[:20]))
        self.counts = {"rows": self.B, "near_draws": near, "exempt_rows": exempt, "sequential_redos": seq,
                       "mismatches_near": near_mismatch}
        return near, near_mismatch


def _rows_view(t):
    """A [B, V] view whose row stride may exceed V (the padded device buffer)."""
    return t
