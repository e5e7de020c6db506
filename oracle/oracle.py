"""ctypes access to the oracle (liboracle.so) and the compiled reference (_ref/libvref.so).

TEST INFRASTRUCTURE ONLY: imported by the tests, the smoke check and the bench's CPU-baseline
leg. The product (verbo_amd) never imports this module.

- ``load_oracle()``: our C restatement of the reference sampler (vsmp_oracle.c).
- ``load_ref()``: the reference's own sampler compiled from its sources (ref_shim.cpp);
  present only where oracle/Makefile could build it.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libvref.so"
REF_TREE = Path("/root/reference")


class Sampling(ctypes.Structure):
    """verbo::Sampling (reference include/verbo/verbo.hpp:56-64), 32 bytes."""

    _fields_ = [
        ("temp", ctypes.c_float),
        ("top_k", ctypes.c_int),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repeat", ctypes.c_float),
        ("repeat_last", ctypes.c_int),
        ("seed", ctypes.c_ulonglong),
    ]


class Info(ctypes.Structure):
    _fields_ = [
        ("id", ctypes.c_int),
        ("greedy", ctypes.c_int),
        ("k", ctypes.c_int),
        ("keep_minp", ctypes.c_int),
        ("keep", ctypes.c_int),
        ("n_pen", ctypes.c_int),
        ("mx", ctypes.c_float),
        ("rank", ctypes.c_int),
        ("last_id", ctypes.c_int),
        ("reserved", ctypes.c_int),
        ("sum", ctypes.c_double),
        ("tot", ctypes.c_double),
        ("u", ctypes.c_double),
        ("minp_margin", ctypes.c_double),
        ("topp_margin", ctypes.c_double),
        ("draw_margin", ctypes.c_double),
    ]


INFO_DTYPE = np.dtype([(n, np.dtype(t)) for n, t in [
    ("id", "i4"), ("greedy", "i4"), ("k", "i4"), ("keep_minp", "i4"), ("keep", "i4"), ("n_pen", "i4"),
    ("mx", "f4"), ("rank", "i4"), ("last_id", "i4"), ("reserved", "i4"), ("sum", "f8"), ("tot", "f8"), ("u", "f8"), ("minp_margin", "f8"),
    ("topp_margin", "f8"), ("draw_margin", "f8")]])
assert INFO_DTYPE.itemsize == ctypes.sizeof(Info)

SAMPLING_DTYPE = np.dtype([("temp", "f4"), ("top_k", "i4"), ("top_p", "f4"), ("min_p", "f4"),
                           ("repeat", "f4"), ("repeat_last", "i4"), ("seed", "u8")])
assert SAMPLING_DTYPE.itemsize == ctypes.sizeof(Sampling) == 32

_P = ctypes.c_void_p
_oracle = None
_ref = None


def build(ref=True):
    """Compile the oracle (and the reference when its tree is present) with oracle/Makefile."""
    targets = ["oracle"]
    if ref and REF_TREE.is_dir():
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", str(HERE), f"-j{min(8, os.cpu_count() or 1)}"] + targets, check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def load_oracle():
    global _oracle
    if _oracle is None:
        if not ORACLE_SO.is_file():
            build(ref=False)
        lib = ctypes.CDLL(str(ORACLE_SO))
        lib.vo_splitmix.restype = ctypes.c_uint64
        lib.vo_splitmix.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        lib.vo_seed.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]
        lib.vo_unit.restype = ctypes.c_double
        lib.vo_unit.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        lib.vo_counter_u.restype = ctypes.c_double
        lib.vo_counter_u.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        lib.vo_accept.restype = ctypes.c_int
        lib.vo_accept.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.vo_pick.restype = ctypes.c_int
        lib.vo_pick.argtypes = [_P, ctypes.c_int, ctypes.POINTER(Sampling), _P, ctypes.c_int, ctypes.c_double,
                                ctypes.POINTER(Info), _P, _P, ctypes.c_int, _P, ctypes.c_int]
        lib.vo_pick_rows.restype = ctypes.c_int
        lib.vo_pick_rows.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_longlong, _P, ctypes.c_int, _P, _P,
                                     _P, _P, _P, _P, _P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_int]
        lib.vo_sampler_run.restype = ctypes.c_int
        lib.vo_sampler_run.argtypes = [_P, ctypes.c_int, ctypes.POINTER(Sampling), _P, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, _P]
        _oracle = lib
    return _oracle


def ref_available():
    return REF_SO.is_file()


def load_ref():
    global _ref
    if _ref is None:
        if not REF_SO.is_file():
            raise FileNotFoundError(f"{REF_SO} is not built (needs the reference tree; run make -C oracle ref)")
        lib = ctypes.CDLL(str(REF_SO))
        lib.vref_sampler_run.restype = ctypes.c_int
        lib.vref_sampler_run.argtypes = [_P, ctypes.c_int, ctypes.POINTER(Sampling), _P, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, _P]
        lib.vref_pick_rows.restype = ctypes.c_int
        lib.vref_pick_rows.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_longlong, _P, ctypes.c_int, _P, _P,
                                       _P, ctypes.c_int]
        lib.vref_sampler_new.restype = ctypes.c_void_p
        lib.vref_sampler_new.argtypes = [ctypes.POINTER(Sampling)]
        lib.vref_sampler_free.argtypes = [ctypes.c_void_p]
        lib.vref_sampler_accept.argtypes = [ctypes.c_void_p, ctypes.c_int]
        lib.vref_sampler_pick.restype = ctypes.c_int
        lib.vref_sampler_pick.argtypes = [ctypes.c_void_p, _P, ctypes.c_int]
        lib.vref_time_rows.restype = ctypes.c_double
        lib.vref_time_rows.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_longlong, _P, ctypes.c_int, _P, _P,
                                       ctypes.c_int, ctypes.c_double, ctypes.POINTER(ctypes.c_longlong)]
        _ref = lib
    return _ref


def sampling(temp=0.7, top_k=40, top_p=0.9, min_p=0.0, repeat=1.0, repeat_last=64, seed=0):
    """A Sampling struct; defaults are the reference's (include/verbo/verbo.hpp:56-64)."""
    return Sampling(temp, top_k, top_p, min_p, repeat, repeat_last, seed)


def params_array(rows):
    """numpy structured array (SAMPLING_DTYPE) from a list of dicts / Sampling structs."""
    out = np.zeros(len(rows), dtype=SAMPLING_DTYPE)
    for i, r in enumerate(rows):
        if isinstance(r, Sampling):
            r = {n: getattr(r, n) for n, _ in Sampling._fields_}
        for n in SAMPLING_DTYPE.names:
            if n in r:
                out[n][i] = r[n]
    return out


# ---- oracle calls -----------------------------------------------------------------------------

def rng_seed(seed):
    st = (ctypes.c_uint64 * 2)()
    load_oracle().vo_seed(seed, st)
    return st


def rng_unit(st):
    return load_oracle().vo_unit(st)


def reference_stream(seed, n):
    """First n uniform draws of a reference Sampler seeded with `seed` (nonzero)."""
    st = rng_seed(seed)
    return np.array([rng_unit(st) for _ in range(n)], dtype=np.float64)


def counter_u(seed, counter):
    return load_oracle().vo_counter_u(seed, counter)


def pick(logits, cfg, hist=(), u=0.0, cand_cap=0, pen_cap=0):
    """One oracle pick. Returns (id, info, cand_ids, cand_pr, pen_ids)."""
    lib = load_oracle()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(hist, dtype=np.int32)
    info = Info()
    cand = np.zeros(max(cand_cap, 1), dtype=np.int32)
    cpr = np.zeros(max(cand_cap, 1), dtype=np.float64)
    pen = np.zeros(max(pen_cap, 1), dtype=np.int32)
    rid = lib.vo_pick(_ptr(lg), lg.size, ctypes.byref(cfg), _ptr(h), h.size, float(u), ctypes.byref(info),
                      _ptr(cand), _ptr(cpr), cand_cap, _ptr(pen), pen_cap)
    m = min(info.keep, cand_cap)
    return rid, info, cand[:m].copy(), cpr[:m].copy(), pen[:min(info.n_pen, pen_cap)].copy()


def pick_rows(logits, params, hist=None, hist_off=None, u=None, cand_cap=0, threads=None, pen_cap=0):
    """Oracle picks for B rows. params: SAMPLING_DTYPE array of 1 (shared) or B entries.
    Returns (ids, infos (INFO_DTYPE), cand [B, cand_cap], cand_pr [B, cand_cap]), and with
    pen_cap > 0 a fifth item: per row, the first pen_cap penalised ids (ascending, int32 arrays)."""
    lib = load_oracle()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = lg.shape
    params = np.ascontiguousarray(params, dtype=SAMPLING_DTYPE)
    per_row = 1 if params.size == B and B > 1 else 0
    if params.size not in (1, B):
        raise ValueError("params must have 1 or B entries")
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    ho = None if hist_off is None else np.ascontiguousarray(hist_off, dtype=np.int32)
    uu = np.zeros(B) if u is None else np.ascontiguousarray(u, dtype=np.float64)
    out = np.zeros(B, dtype=np.int32)
    infos = np.zeros(B, dtype=INFO_DTYPE)
    cand = np.zeros((B, max(cand_cap, 1)), dtype=np.int32) if cand_cap else None
    cpr = np.zeros((B, max(cand_cap, 1)), dtype=np.float64) if cand_cap else None
    pen = np.zeros((B, pen_cap), dtype=np.int32) if pen_cap else None
    threads = threads or min(8, os.cpu_count() or 1)
    lib.vo_pick_rows(_ptr(lg), B, V, V, _ptr(params), per_row, _ptr(h), _ptr(ho), _ptr(uu), _ptr(out),
                     _ptr(infos), _ptr(cand), _ptr(cpr), cand_cap, _ptr(pen), pen_cap, threads)
    if not pen_cap:
        return out, infos, cand, cpr
    return out, infos, cand, cpr, [pen[r, :min(int(infos["n_pen"][r]), pen_cap)].copy() for r in range(B)]


def sampler_run(logits, cfg, hist=(), n_picks=1, accept_each=False):
    """Oracle Sampler run (seeded xorshift stream), see vo_sampler_run."""
    lib = load_oracle()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(hist, dtype=np.int32)
    out = np.zeros(n_picks, dtype=np.int32)
    rc = lib.vo_sampler_run(_ptr(lg), lg.size, ctypes.byref(cfg), _ptr(h), h.size, n_picks, int(accept_each),
                            _ptr(out))
    if rc != 0:
        raise ValueError("vo_sampler_run: bad input (seed must be nonzero)")
    return out


# ---- compiled-reference calls -----------------------------------------------------------------

def ref_sampler_run(logits, cfg, hist=(), n_picks=1, accept_each=False):
    lib = load_ref()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(hist, dtype=np.int32)
    out = np.zeros(n_picks, dtype=np.int32)
    lib.vref_sampler_run(_ptr(lg), lg.size, ctypes.byref(cfg), _ptr(h), h.size, n_picks, int(accept_each),
                         _ptr(out))
    return out


def ref_pick_rows(logits, params, hist=None, hist_off=None, threads=None):
    lib = load_ref()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = lg.shape
    params = np.ascontiguousarray(params, dtype=SAMPLING_DTYPE)
    per_row = 1 if params.size == B and B > 1 else 0
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    ho = None if hist_off is None else np.ascontiguousarray(hist_off, dtype=np.int32)
    out = np.zeros(B, dtype=np.int32)
    lib.vref_pick_rows(_ptr(lg), B, V, V, _ptr(params), per_row, _ptr(h), _ptr(ho), _ptr(out),
                       threads or min(8, os.cpu_count() or 1))
    return out


def ref_time_rows(logits, params, hist=None, hist_off=None, threads=1, budget_s=10.0):
    """Wall-clock pick() throughput of the compiled reference. Returns (seconds, picks)."""
    lib = load_ref()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = lg.shape
    params = np.ascontiguousarray(params, dtype=SAMPLING_DTYPE)
    per_row = 1 if params.size == B and B > 1 else 0
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    ho = None if hist_off is None else np.ascontiguousarray(hist_off, dtype=np.int32)
    n = ctypes.c_longlong(0)
    s = lib.vref_time_rows(_ptr(lg), B, V, V, _ptr(params), per_row, _ptr(h), _ptr(ho), threads, budget_s,
                           ctypes.byref(n))
    return s, n.value


class RefSampler:
    """A reference verbo::Sampler (compiled from its sources) behind a handle: pick / accept."""

    def __init__(self, cfg):
        self._lib = load_ref()
        self._h = self._lib.vref_sampler_new(ctypes.byref(cfg))

    def pick(self, logits):
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        return self._lib.vref_sampler_pick(self._h, _ptr(lg), lg.size)

    def accept(self, tok):
        self._lib.vref_sampler_accept(self._h, int(tok))

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.vref_sampler_free(self._h)
            self._h = None
