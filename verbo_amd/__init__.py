"""verbo's token sampler on AMD Instinct MI355X: Python bindings of libvsmp.so (include/vsmp.h).

Mirrors the reference's ctypes layer (python/verbo/__init__.py): a library loader that honours
an environment override, a parameter struct laid out like verbo::Sampling, errors raised from
the library's per-thread message. Device buffers are torch tensors on a ROCm device; only their
addresses cross the C ABI.

    ctx = Context()
    ids = ctx.pick_batch(logits, Params(temp=.8, top_k=50), u_mode=U_COUNTER)  # logits: cuda [B,V]
    s = Sampler(temp=.7, seed=42); s.accept(3); tok = s.pick(numpy_row)        # verbo::Sampler
"""
import ctypes
import os
from pathlib import Path

import numpy as np

from .workloads import SAMPLING_DTYPE

__all__ = ["Context", "Sampler", "Params", "RowInfo", "Debug", "VsmpError", "pick_batch_noalloc", "load_library", "U_SUPPLIED", "U_COUNTER",
           "U_XORSHIFT", "ROW_INFO_DTYPE", "SAMPLING_DTYPE"]
__version__ = "0.1.0"

U_SUPPLIED, U_COUNTER, U_XORSHIFT = 0, 1, 2
FLAG_TOPP_NEAR, FLAG_MINP_NEAR, FLAG_DRAW_NEAR, FLAG_FALLBACK = 1, 2, 4, 8
FLAG_SEQ_CUTS, FLAG_CUTS_DIFFER = 16, 32
FLAG_ONE_PASS, FLAG_MINP_PREFIX = 64, 128
PATH_GREEDY, PATH_SMALLK, PATH_GENERAL = 0, 1, 2


class VsmpError(RuntimeError):
    pass


class Params(ctypes.Structure):
    """vsmp_params == verbo::Sampling (reference include/verbo/verbo.hpp:56-64); defaults are the
    reference's."""

    _fields_ = [
        ("temp", ctypes.c_float),
        ("top_k", ctypes.c_int),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repeat", ctypes.c_float),
        ("repeat_last", ctypes.c_int),
        ("seed", ctypes.c_ulonglong),
    ]

    def __init__(self, temp=0.7, top_k=40, top_p=0.9, min_p=0.0, repeat=1.0, repeat_last=64, seed=0):
        super().__init__(temp, top_k, top_p, min_p, repeat, repeat_last, seed)


class RowInfo(ctypes.Structure):
    _fields_ = [
        ("id", ctypes.c_int),
        ("path", ctypes.c_int),
        ("k", ctypes.c_int),
        ("keep_minp", ctypes.c_int),
        ("keep", ctypes.c_int),
        ("rank", ctypes.c_int),
        ("last_id", ctypes.c_int),
        ("flags", ctypes.c_int),
        ("mx", ctypes.c_float),
        ("n_pen", ctypes.c_int),
        ("sum", ctypes.c_double),
        ("tot", ctypes.c_double),
        ("u", ctypes.c_double),
        ("draw_margin", ctypes.c_double),
    ]


class Debug(ctypes.Structure):
    """vsmp_debug: optional diagnostic outputs of vsmp_pick_batch (device addresses)."""

    _fields_ = [
        ("info", ctypes.c_void_p),
        ("cand_ids", ctypes.c_void_p),
        ("cand_pr", ctypes.c_void_p),
        ("cand_cap", ctypes.c_int),
        ("pen_bits", ctypes.c_void_p),
    ]


ROW_INFO_DTYPE = np.dtype([("id", "i4"), ("path", "i4"), ("k", "i4"), ("keep_minp", "i4"), ("keep", "i4"),
                           ("rank", "i4"), ("last_id", "i4"), ("flags", "i4"), ("mx", "f4"), ("n_pen", "i4"),
                           ("sum", "f8"), ("tot", "f8"), ("u", "f8"), ("draw_margin", "f8")])
assert ROW_INFO_DTYPE.itemsize == ctypes.sizeof(RowInfo) == 72
assert SAMPLING_DTYPE.itemsize == ctypes.sizeof(Params) == 32

_lib = None
_P = ctypes.c_void_p


def _candidates():
    env = os.environ.get("VSMP_LIB")
    if env:
        yield Path(env)
    yield Path(__file__).resolve().parent / "libvsmp.so"


def load_library():
    """Load libvsmp.so (VSMP_LIB overrides the in-tree path). Raises VsmpError if it is missing:
    there is no fallback implementation."""
    global _lib
    if _lib is not None:
        return _lib
    # torch ships its own HIP runtime under the same soname (libamdhip64.so.7). Whichever loads
    # first serves the whole process, and torch cannot use a newer one; so when torch is present
    # it is loaded first and this library, its kernels and torch's streams share its runtime.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    for p in _candidates():
        if p.is_file():
            lib = ctypes.CDLL(str(p))
            break
    else:
        raise VsmpError("libvsmp.so not found; build it with `python -m verbo_amd.build` or set VSMP_LIB")
    sig = {
        "vsmp_last_error": (ctypes.c_char_p, []),
        "vsmp_version": (ctypes.c_char_p, []),
        "vsmp_ctx_new": (_P, [ctypes.c_int]),
        "vsmp_ctx_free": (None, [_P]),
        "vsmp_pick_batch": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_longlong, _P, ctypes.c_int,
                                           _P, _P, ctypes.c_int, _P, _P, ctypes.c_ulonglong, _P,
                                           ctypes.POINTER(Debug), _P]),
        "vsmp_pick_batch_noalloc": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_longlong, _P, ctypes.c_int,
                                                   _P, _P, ctypes.c_int, _P, _P, ctypes.c_ulonglong, _P,
                                                   ctypes.POINTER(Debug), _P]),
        "vsmp_pick_host": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.POINTER(Params), _P, ctypes.c_int,
                                          ctypes.c_double, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(RowInfo)]),
        "vsmp_sampler_new": (_P, [ctypes.POINTER(Params)]),
        "vsmp_sampler_free": (None, [_P]),
        "vsmp_sampler_pick": (ctypes.c_int, [_P, _P, ctypes.c_int]),
        "vsmp_sampler_accept": (None, [_P, ctypes.c_int]),
        "vsmp_sampler_reset": (None, [_P]),
        "vsmp_read_probe": (ctypes.c_int, [_P, _P, ctypes.c_longlong, _P]),
        "vsmp_exp_probe": (ctypes.c_int, [_P, _P, _P, ctypes.c_longlong, _P]),
        "vsmp_numer_probe": (ctypes.c_int, [_P, _P, _P, ctypes.c_longlong, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                            _P]),
        "vsmp_head_logits": (ctypes.c_int, [_P, _P, ctypes.c_longlong, _P, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _P, ctypes.c_longlong, _P]),
        "vsmp_head_pick": (ctypes.c_int, [_P, _P, ctypes.c_longlong, _P, ctypes.c_longlong, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, _P, ctypes.c_int, _P, _P, ctypes.c_int, _P, _P,
                                          ctypes.c_ulonglong, _P, _P, ctypes.c_longlong, ctypes.POINTER(Debug), _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _err():
    return VsmpError(_lib.vsmp_last_error().decode("utf-8", "replace"))


def version():
    return load_library().vsmp_version().decode()


def _addr(t):
    """Device address of a torch tensor (None stays None)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise VsmpError("expected a device tensor")
    if not t.is_contiguous():
        raise VsmpError("expected a contiguous tensor")
    return t.data_ptr()


DEFAULTS = {"temp": 0.7, "top_k": 40, "top_p": 0.9, "min_p": 0.0, "repeat": 1.0, "repeat_last": 64, "seed": 0}


def params_array(rows=None, n=None, **fields):
    """A SAMPLING_DTYPE array: from a list of dicts/Params, or `n` copies of the given fields
    (missing fields take the reference's defaults)."""
    if rows is None:
        rows = [fields] * int(n or 1)
    out = np.zeros(len(rows), dtype=SAMPLING_DTYPE)
    for i, r in enumerate(rows):
        if isinstance(r, Params):
            r = {f: getattr(r, f) for f, _ in Params._fields_}
        d = dict(DEFAULTS, **r)
        for f in SAMPLING_DTYPE.names:
            out[f][i] = d[f]
    return out


def to_device_params(arr, device="cuda"):
    """Upload a SAMPLING_DTYPE array as a device byte tensor for per-row parameters."""
    import torch

    a = np.ascontiguousarray(arr, dtype=SAMPLING_DTYPE)
    return torch.from_numpy(a.view(np.uint8).copy()).to(device)


def row_info(t):
    """Host numpy ROW_INFO_DTYPE view of a device info tensor (uint8, B*72 bytes)."""
    return t.cpu().numpy().view(ROW_INFO_DTYPE)


def pen_ids(bits, V):
    """Ascending penalised ids per row from a pen_bits bitmap (numpy int32 [B, ceil(V/32)])."""
    b = np.ascontiguousarray(bits).view(np.uint32)
    flat = np.unpackbits(b.view(np.uint8).reshape(b.shape[0], -1), axis=1, bitorder="little")[:, :V]
    return [np.nonzero(r)[0].astype(np.int32) for r in flat]


def _batch_args(logits, params, hist, hist_off, u_mode, u, rng_state, counter, out, info, cand_ids, cand_pr, pen_bits,
                stream):
    """The arguments of vsmp_pick_batch after the context, the output tensor, and the objects whose
    addresses the arguments hold (kept alive by the caller until the call returns)."""
    import torch

    if logits.dim() != 2 or logits.dtype != torch.float32:
        raise VsmpError("logits must be a 2-D float32 device tensor")
    if not logits.is_cuda:
        raise VsmpError("logits must be a device tensor")
    B, V = logits.shape
    ld = logits.stride(0)
    if logits.stride(1) != 1:
        raise VsmpError("logits rows must be contiguous")
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    if isinstance(params, Params):
        pp, per_row = ctypes.addressof(params), 0
    else:
        if params.numel() != 32 * B:
            raise VsmpError("per-row params must hold B entries")
        pp, per_row = _addr(params), 1
    cap = cand_ids.shape[1] if cand_ids is not None else 0
    if pen_bits is not None and pen_bits.numel() != B * ((V + 31) // 32):
        raise VsmpError("pen_bits must hold B * ceil(V / 32) words")
    dbg = None
    if info is not None or cand_ids is not None or pen_bits is not None:
        dbg = Debug(_addr(info), _addr(cand_ids), _addr(cand_pr), cap, _addr(pen_bits))
    st = stream if stream is not None else torch.cuda.current_stream(logits.device)
    args = (logits.data_ptr(), B, V, ld, pp, per_row, _addr(hist), _addr(hist_off), int(u_mode), _addr(u),
            _addr(rng_state), int(counter), _addr(out), ctypes.byref(dbg) if dbg is not None else None,
            ctypes.c_void_p(st.cuda_stream))
    return args, out, (params, dbg)


def pick_batch_noalloc(logits, params, hist=None, hist_off=None, u_mode=U_COUNTER, u=None, rng_state=None, counter=0,
                       out=None, info=None, cand_ids=None, cand_pr=None, pen_bits=None, stream=None):
    """vsmp_pick_batch_noalloc: Context.pick_batch's call without a context and without allocating
    (row mode; B <= 2048, V <= 262144; the scratch is a static device array shared by every call on
    the GPU, so calls must not overlap)."""
    load_library()
    args, out, keep = _batch_args(logits, params, hist, hist_off, u_mode, u, rng_state, counter, out, info, cand_ids,
                                  cand_pr, pen_bits, stream)
    if _lib.vsmp_pick_batch_noalloc(*args) != 0:
        raise _err()
    del keep
    return out


def _check_rows(t, dtype, name):
    if not t.is_cuda or t.dtype != dtype or t.dim() != 2 or t.stride(1) != 1:
        raise VsmpError(f"{name} must be a 2-D {dtype} device tensor with contiguous rows")


def _head_shapes(hidden, head):
    """(B, D, V) of a head call on bf16 device tensors hidden [B, D] and head [V, D]."""
    import torch

    _check_rows(hidden, torch.bfloat16, "hidden")
    _check_rows(head, torch.bfloat16, "head")
    if hidden.shape[1] != head.shape[1]:
        raise VsmpError("hidden and head must have the same number of columns (D)")
    return hidden.shape[0], hidden.shape[1], head.shape[0]


class Context:
    """A vsmp_ctx on one device: scratch for batched picks, staging for host picks."""

    def __init__(self, device=0):
        load_library()
        self._h = _lib.vsmp_ctx_new(int(device))
        if not self._h:
            raise _err()
        self.device = device

    def close(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.vsmp_ctx_free(h)
            self._h = None

    def __del__(self):
        self.close()

    def pick_batch(self, logits, params, hist=None, hist_off=None, u_mode=U_COUNTER, u=None, rng_state=None,
                   counter=0, out=None, info=None, cand_ids=None, cand_pr=None, pen_bits=None, stream=None):
        """vsmp_pick_batch on torch device tensors. `params`: a Params (shared by all rows) or a
        device byte tensor from to_device_params (one entry per row). Returns `out` (int32 [B]).
        Diagnostics (vsmp_debug): info (uint8 [B*72]), cand_ids (int32 [B, cap]) / cand_pr (float64
        [B, cap]), pen_bits (int32 [B, ceil(V/32)]).
        Stream-ordered on `stream` (default: torch's current stream); does not synchronise."""
        args, out, keep = _batch_args(logits, params, hist, hist_off, u_mode, u, rng_state, counter, out, info,
                                      cand_ids, cand_pr, pen_bits, stream)
        if _lib.vsmp_pick_batch(self._h, *args) != 0:
            raise _err()
        del keep
        return out

    def head_logits(self, hidden, head, logits=None, stream=None):
        """vsmp_head_logits: logits = hidden @ head.T for bf16 device tensors hidden [B, D] and head
        [V, D] (rows contiguous), fp32 accumulation; returns logits (float32 [B, V] unless given)."""
        import torch

        B, D, V = _head_shapes(hidden, head)
        if logits is None:  # rows padded to 16 bytes, so that pick_batch can take them
            logits = torch.empty(B, (V + 3) // 4 * 4, dtype=torch.float32, device=hidden.device)[:, :V]
        _check_rows(logits, torch.float32, "logits")
        st = stream if stream is not None else torch.cuda.current_stream(hidden.device)
        if _lib.vsmp_head_logits(self._h, hidden.data_ptr(), hidden.stride(0), head.data_ptr(), head.stride(0), B, V, D,
                                 logits.data_ptr(), logits.stride(0), ctypes.c_void_p(st.cuda_stream)) != 0:
            raise _err()
        return logits

    def head_pick(self, hidden, head, params, hist=None, hist_off=None, u_mode=U_COUNTER, u=None, rng_state=None,
                  counter=0, out=None, logits=None, info=None, cand_ids=None, cand_pr=None, pen_bits=None, stream=None):
        """vsmp_head_pick: the head's product and pick_batch's pick in one call (the ids pick_batch
        takes from head_logits' logits). `logits`: None, or a float32 [B, >= V] device tensor that
        receives the logits as well. The rest as pick_batch. Returns `out` (int32 [B])."""
        import torch

        B, D, V = _head_shapes(hidden, head)
        if out is None:
            out = torch.empty(B, dtype=torch.int32, device=hidden.device)
        if logits is not None:
            _check_rows(logits, torch.float32, "logits")
        if isinstance(params, Params):
            pp, per_row = ctypes.addressof(params), 0
        else:
            if params.numel() != 32 * B:
                raise VsmpError("per-row params must hold B entries")
            pp, per_row = _addr(params), 1
        cap = cand_ids.shape[1] if cand_ids is not None else 0
        if pen_bits is not None and pen_bits.numel() != B * ((V + 31) // 32):
            raise VsmpError("pen_bits must hold B * ceil(V / 32) words")
        dbg = None
        if info is not None or cand_ids is not None or pen_bits is not None:
            dbg = Debug(_addr(info), _addr(cand_ids), _addr(cand_pr), cap, _addr(pen_bits))
        st = stream if stream is not None else torch.cuda.current_stream(hidden.device)
        rc = _lib.vsmp_head_pick(self._h, hidden.data_ptr(), hidden.stride(0), head.data_ptr(), head.stride(0), B, V, D,
                                 pp, per_row, _addr(hist), _addr(hist_off), int(u_mode), _addr(u), _addr(rng_state),
                                 int(counter), _addr(out), logits.data_ptr() if logits is not None else None,
                                 logits.stride(0) if logits is not None else 0,
                                 ctypes.byref(dbg) if dbg is not None else None, ctypes.c_void_p(st.cuda_stream))
        if rc != 0:
            raise _err()
        del params, dbg
        return out

    def read_probe(self, t, stream=None):
        """vsmp_read_probe: stream the bytes of device tensor `t` through a plain read kernel on
        `stream` (default: torch's current stream). For measuring attainable read bandwidth."""
        import torch

        st = stream if stream is not None else torch.cuda.current_stream(t.device)
        nbytes = t.numel() * t.element_size() // 16 * 16
        if _lib.vsmp_read_probe(self._h, t.data_ptr(), nbytes, ctypes.c_void_p(st.cuda_stream)) != 0:
            raise _err()

    def exp_probe(self, x, stream=None):
        """vsmp_exp_probe: the general path's fp64 exp over device tensor `x` (float64); returns y."""
        import torch

        if x.dtype != torch.float64 or not x.is_cuda:
            raise VsmpError("exp_probe needs a float64 device tensor")
        x = x.contiguous()
        y = torch.empty_like(x)
        st = stream if stream is not None else torch.cuda.current_stream(x.device)
        if _lib.vsmp_exp_probe(self._h, x.data_ptr(), y.data_ptr(), x.numel(), ctypes.c_void_p(st.cuda_stream)) != 0:
            raise _err()
        return y

    def numer_probe(self, d, temp, qs, fixed_point=False, stream=None):
        """vsmp_numer_probe: the general path's numerators exp(double(d) / temp) for float32 device
        tensor `d` (= v - max <= 0), buckets of scale qs: the table numerators, or with fixed_point
        each element's share of its bucket's mass; returns float64 y."""
        import torch

        if d.dtype != torch.float32 or not d.is_cuda:
            raise VsmpError("numer_probe needs a float32 device tensor")
        d = d.contiguous()
        y = torch.empty(d.shape, dtype=torch.float64, device=d.device)
        st = stream if stream is not None else torch.cuda.current_stream(d.device)
        if _lib.vsmp_numer_probe(self._h, d.data_ptr(), y.data_ptr(), d.numel(), float(temp), float(qs),
                                 1 if fixed_point else 0, ctypes.c_void_p(st.cuda_stream)) != 0:
            raise _err()
        return y

    def pick_host(self, logits, params, hist=(), u=0.0, with_info=False):
        """vsmp_pick_host: one pick on a host row (numpy). Returns id (and RowInfo)."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        h = np.ascontiguousarray(hist, dtype=np.int32)
        out = ctypes.c_int(-1)
        info = RowInfo()
        rc = _lib.vsmp_pick_host(self._h, lg.ctypes.data_as(_P), lg.size, ctypes.byref(params),
                                 h.ctypes.data_as(_P) if h.size else None, h.size, float(u), ctypes.byref(out),
                                 ctypes.byref(info) if with_info else None)
        if rc != 0:
            raise _err()
        return (out.value, info) if with_info else out.value


class Sampler:
    """verbo::Sampler (reference include/verbo/verbo.hpp:116-132) with pick on the GPU."""

    def __init__(self, params=None, **kw):
        load_library()
        p = params if params is not None else Params(**kw)
        self._h = _lib.vsmp_sampler_new(ctypes.byref(p))
        if not self._h:
            raise _err()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.vsmp_sampler_free(h)
            self._h = None

    def pick(self, logits):
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        # the address as a plain int: ndarray.ctypes.data_as builds several objects per call
        r = _lib.vsmp_sampler_pick(self._h, lg.ctypes.data, lg.size)
        if r < 0:
            raise _err()
        return r

    def accept(self, tok):
        _lib.vsmp_sampler_accept(self._h, int(tok))

    def reset(self):
        _lib.vsmp_sampler_reset(self._h)
