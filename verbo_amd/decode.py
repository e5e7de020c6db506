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

A server keeps a decoder of a fixed number of slots and lets requests take them as they arrive and
free them as they finish (continuous batching); each step samples only the live slots:

    dec = BatchDecoder.with_slots(8, vocab=V)
    res = dec.serve([Request(prompt, Opts(max_tokens=32, seed=7), arrival=3), ...], logits_fn, stop_ids={2})
    # logits_fn(reqs, steps, last) -> cuda [len(reqs), V]: each live request's next position

`Opts` mirrors the reference's option block (`_Opts`, python/verbo/__init__.py:16-25, the C ABI's
verbo_gen_opts): the fields verbo_generate lets a caller set. Like verbo_generate, which keeps the
model's repeat_last (src/capi.cpp:131-151), BatchDecoder takes repeat_last (default 64) apart.
"""
import ctypes

import numpy as np

from . import Params, VsmpError, _err, load_library

__all__ = ["Opts", "Request", "BatchDecoder", "params_of"]


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


class Request:
    """One generation request of a serving loop: the prompt's ids, its options (Opts), the window
    of its repetition penalty and the step at which it arrives."""

    def __init__(self, prompt, opts, repeat_last=64, arrival=0):
        self.prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        self.opts = opts
        self.repeat_last = int(repeat_last)
        self.arrival = int(arrival)


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
            "vsmp_bsampler_admit": (ctypes.c_int, [P, ctypes.c_int, P, P, ctypes.c_int, P]),
            "vsmp_bsampler_pick_rows": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_longlong, P, ctypes.c_int, P, P]),
            "vsmp_bsampler_accept_rows": (ctypes.c_int, [P, P, P, P, ctypes.c_int, P]),
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
        stopped): the ids generated and whether a stop id ended the sequence. Sequence r decodes in
        slot r with the options given at construction; each step samples the live rows only (serve()
        with every request arriving at step 0)."""
        import torch

        rl = [int(p.repeat_last) for p in self.params]
        reqs = [Request(p, o, r, 0) for p, o, r in zip(prompts, self.opts, rl)]
        n = self.n

        def rows_of(js, steps, last):
            # every live sequence was admitted at step 0 and picked at every step since: one step for all
            last_all = np.full(n, -1, np.int64)
            last_all[js] = last
            live = np.zeros(n, bool)
            live[js] = True
            lg = logits_fn(int(steps[0]), last_all, live)
            return lg.index_select(0, torch.as_tensor(js, dtype=torch.long, device=lg.device))

        return self.serve(reqs, rows_of, stop_ids)

    @classmethod
    def with_slots(cls, slots, vocab, cap=4096, device=0):
        """A decoder of `slots` slots for serve(): every slot free until a request takes it.
        cap: history ids a slot holds (at least 4 * repeat_last of every request admitted)."""
        return cls([Opts(max_tokens=0, temp=0.0)] * int(slots), vocab, repeat_last=0, cap=cap, device=device)

    def admit(self, slot, params, prompt, stream):
        """vsmp_bsampler_admit: a new sequence (verbo::Sampler(params) that accepted `prompt`) takes
        `slot`, ordered on `stream` after the slot's earlier work."""
        a = np.ascontiguousarray(prompt, dtype=np.int32)
        if self.lib.vsmp_bsampler_admit(self._h, int(slot), ctypes.byref(params), a.ctypes.data if a.size else None,
                                        int(a.size), ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise _err()

    def pick_rows(self, logits, rows, out, stream):
        """One pick for each live slot rows[i] (device int32) from device logits [len(rows), V]."""
        n = int(rows.numel())
        if logits.shape != (n, self.vocab) or logits.stride(1) != 1:
            raise VsmpError("logits must be a [len(rows), V] device tensor with contiguous rows")
        if self.lib.vsmp_bsampler_pick_rows(self._h, logits.data_ptr(), self.vocab, logits.stride(0), rows.data_ptr(), n,
                                            out.data_ptr(), ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise _err()

    def accept_rows(self, ids, rows, active, stream):
        """Sampler::accept of ids[i] into slot rows[i] where active[i] != 0 (device int32 tensors)."""
        if self.lib.vsmp_bsampler_accept_rows(self._h, ids.data_ptr(), rows.data_ptr(), active.data_ptr(),
                                              int(rows.numel()), ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise _err()

    def serve(self, requests, logits_fn, stop_ids=()):
        """Continuous batching over the decoder's slots: each step, requests that have arrived take
        free slots (in arrival order, the lowest slot first), then every live slot is sampled at once
        and only the live slots: logits_fn(reqs, steps, last) returns the device logits
        [len(reqs), V] of the requests reqs (indices into `requests`) at their own steps `steps`
        after their last ids `last` (-1 before a request's first pick). Per request, the semantics
        are those of verbo::generate (reference src/sampler.cpp:111-181; cli/serve.cpp:139-192 runs
        it per request): the prompt accepted first, a stop id ends the sequence unaccepted, any other
        id is accepted and counted until max_tokens. A finished request's slot is free for the next
        step. Returns per request (tokens, stopped); self.schedule holds per step the (request,
        slot) pairs that were sampled."""
        import torch

        stops = set(int(x) for x in stop_ids)
        dev = torch.device("cuda", self.device)
        stream = torch.cuda.current_stream(dev)
        out = torch.empty(self.n, dtype=torch.int32, device=dev)
        order = sorted(range(len(requests)), key=lambda j: (requests[j].arrival, j))
        queue = list(order)
        free = list(range(self.n))
        live = {}  # slot -> request
        toks = [[] for _ in requests]
        stopped = [False] * len(requests)
        steps = [0] * len(requests)
        last = [-1] * len(requests)
        self.schedule = []
        step = 0
        while queue or live:
            while queue and requests[queue[0]].arrival <= step and free:
                j = queue.pop(0)
                r = requests[j]
                if r.opts.max_tokens <= 0:
                    continue  # nothing to generate: done without a slot
                slot = free.pop(0)
                self.admit(slot, params_of(r.opts, r.repeat_last), r.prompt, stream)
                live[slot] = j
            if not live:
                step += 1
                continue
            slots = sorted(live)
            reqs = [live[s] for s in slots]
            rows = torch.tensor(slots, dtype=torch.int32, device=dev)
            self.pick_rows(logits_fn(reqs, [steps[j] for j in reqs], [last[j] for j in reqs]), rows,
                           out[:len(slots)], stream)
            self.schedule.append(list(zip(reqs, slots)))
            ids = out[:len(slots)].cpu().numpy()  # the only per-step copy to the host: one id per live slot
            take = np.zeros(len(slots), np.int32)
            done = []
            for i, (s, j) in enumerate(zip(slots, reqs)):
                t = int(ids[i])
                steps[j] += 1
                if t in stops:  # not accepted, not counted (src/sampler.cpp:159-162)
                    stopped[j] = True
                    done.append(s)
                    continue
                take[i] = 1
                toks[j].append(t)
                last[j] = t
                if len(toks[j]) >= requests[j].opts.max_tokens:
                    done.append(s)
            self.accept_rows(out[:len(slots)], rows, torch.from_numpy(take).to(dev), stream)
            for s in done:
                del live[s]
                free.append(s)
            free.sort()
            step += 1
        if self.lib.vsmp_bsampler_full(self._h, ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise VsmpError("a sequence's history outgrew its slot's region (cap)")
        return list(zip(toks, stopped))
