"""Batched decoding on the GPU: N sequences picked together, each with its own sampling options,
their draw streams and history windows on the device (vsmp_bsampler in include/vsmp.h).

The reference serves one request at a time (cli/serve.cpp:168) and binds one verbo_generate per
session (python/verbo/__init__.py:206-236). Here a continuous-batching step picks for every live
sequence at once from [N x V] device logits: per sequence the semantics are those of
verbo::generate's loop (reference src/sampler.cpp:111-181) — the prompt is accepted into the
history, a stop id ends the sequence without being accepted, every other id is accepted and
counted until max_tokens. Only the N picked ids come back to the host each step, for the stop
check; the accepts happen on the device.

    dec = BatchDecoder([Opts(max_tokens=64, temp=0.8, seed=1), Opts(temp=0.0)], vocab=V)
    toks = dec.generate(prompts, logits_fn, stop_ids={2})   # logits_fn(step, last, live) -> cuda [N, V]

`Opts` mirrors the reference's option block (`_Opts`, python/verbo/__init__.py:16-25, the C ABI's
verbo_gen_opts): the fields verbo_generate lets a caller set. Like verbo_generate, which keeps the
model's repeat_last (src/capi.cpp:131-151), BatchDecoder takes repeat_last (default 64) apart.
"""
import ctypes

import numpy as np

from . import Params, VsmpError, _err, load_library

__all__ = ["Opts", "BatchDecoder", "params_of"]


class Opts(ctypes.Structure):
    """verbo_gen_opts (reference include/verbo/verbo.h; python/verbo/__init__.py:16-25 `_Opts`)."""

    _fields_ = [
        ("max_tokens", ctypes.c_int),
        ("temp", ctypes.c_float),
        ("top_k", ctypes.c_int),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repeat", ctypes.c_float),
        ("seed", ctypes.c_ulonglong),
    ]

    def __init__(self, max_tokens=256, temp=0.7, top_k=40, top_p=0.9, min_p=0.0, repeat=1.0, seed=0):
        super().__init__(max_tokens, temp, top_k, top_p, min_p, repeat, seed)


def params_of(o, repeat_last=64):
    """The verbo::Sampling that verbo_generate builds from an option block (src/capi.cpp:136-146)."""
    return Params(o.temp, o.top_k, o.top_p, o.min_p, o.repeat, repeat_last, o.seed)


_sig_done = False


def _lib():
    global _sig_done
    lib = load_library()
    if not _sig_done:
        P = ctypes.c_void_p
        for name, (res, args) in {
            "vsmp_bsampler_new": (P, [ctypes.c_int, ctypes.c_int, P, ctypes.c_int]),
            "vsmp_bsampler_free": (None, [P]),
            "vsmp_bsampler_accept_host": (ctypes.c_int, [P, ctypes.c_int, P, ctypes.c_int]),
            "vsmp_bsampler_pick": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_longlong, P, P]),
            "vsmp_bsampler_accept": (ctypes.c_int, [P, P, P, P]),
            "vsmp_bsampler_full": (ctypes.c_int, [P, P]),
        }.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _sig_done = True
    return lib


class BatchDecoder:
    """N sequences decoded together on one device (vsmp_bsampler).

    opts: one Opts per sequence. cap: history ids each sequence may hold (at least 4 * repeat_last;
    default: that, or, with repeat_last <= 0, the longest prompt plus max_tokens must fit)."""

    def __init__(self, opts, vocab, repeat_last=64, cap=None, device=0):
        self.lib = _lib()
        self.opts = list(opts)
        self.n = len(self.opts)
        self.vocab = int(vocab)
        self.device = device
        rl = repeat_last if np.ndim(repeat_last) else [repeat_last] * self.n
        self.params = (Params * self.n)(*[params_of(o, int(r)) for o, r in zip(self.opts, rl)])
        need = max([4 * int(r) for r in rl if int(r) > 0] + [1])
        self.cap = int(cap) if cap is not None else max(need, 4096)
        self._h = self.lib.vsmp_bsampler_new(int(device), self.n, ctypes.cast(self.params, ctypes.c_void_p), self.cap)
        if not self._h:
            raise _err()

    def close(self):
        if getattr(self, "_h", None):
            self.lib.vsmp_bsampler_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def accept_prompt(self, row, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        if self.lib.vsmp_bsampler_accept_host(self._h, int(row), a.ctypes.data_as(ctypes.c_void_p) if a.size else None,
                                             int(a.size)) != 0:
            raise _err()

    def pick(self, logits, out, stream):
        """One pick per sequence from device logits [N, V] (rows may be strided) into device out[N]."""
        if logits.shape != (self.n, self.vocab) or logits.stride(1) != 1:
            raise VsmpError("logits must be a [N, V] device tensor with contiguous rows")
        if self.lib.vsmp_bsampler_pick(self._h, logits.data_ptr(), self.vocab, logits.stride(0), out.data_ptr(),
                                       ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise _err()

    def accept(self, ids, live, stream):
        """Sampler::accept of ids[r] for every row with live[r] != 0 (device int32 tensors)."""
        if self.lib.vsmp_bsampler_accept(self._h, ids.data_ptr(), live.data_ptr(),
                                         ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise _err()

    def generate(self, prompts, logits_fn, stop_ids=()):
        """Decodes every sequence to its end: per step, logits_fn(step, last, live) returns the device
        logits [N, V] of the next position of every row (last: each row's last id, or -1 before its
        first pick; live: which rows still decode, a host bool array). Returns per row (tokens,
        stopped): the ids generated and whether a stop id ended the sequence."""
        import torch

        stops = set(int(s) for s in stop_ids)
        for r, p in enumerate(prompts):
            self.accept_prompt(r, p)
        dev = torch.device("cuda", self.device)
        stream = torch.cuda.current_stream(dev)
        out = torch.empty(self.n, dtype=torch.int32, device=dev)
        toks = [[] for _ in range(self.n)]
        stopped = [False] * self.n
        live = np.array([o.max_tokens > 0 for o in self.opts])
        last = np.full(self.n, -1, np.int64)
        step = 0
        while live.any():
            self.pick(logits_fn(step, last.copy(), live.copy()), out, stream)
            ids = out.cpu().numpy()  # the only per-step copy to the host: N ids
            take = np.zeros(self.n, np.int32)
            for r in np.flatnonzero(live):
                t = int(ids[r])
                if t in stops:  # not accepted, not counted (src/sampler.cpp:159-162)
                    live[r] = False
                    stopped[r] = True
                    continue
                take[r] = 1
                toks[r].append(t)
                last[r] = t
                if len(toks[r]) >= self.opts[r].max_tokens:
                    live[r] = False
            self.accept(out, torch.from_numpy(take).to(dev), stream)
            step += 1
        if self.lib.vsmp_bsampler_full(self._h, ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise VsmpError("a sequence's history outgrew its region (cap)")
        return list(zip(toks, stopped))
