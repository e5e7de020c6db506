"""Seeded synthetic sampler workloads (logits, histories, per-row parameters).

Everything is drawn from one counter-based generator: output n of a SplitMix64 stream
(x_n = mix(seed + (n+1)*0x9E3779B97F4A7C15)), so any slice of any stream can be regenerated
independently, on any host, with plain numpy. Normals are Box-Muller in fp64 rounded to fp32,
Gumbel(0,1) is -ln(-ln U).

Workloads (B rows x V vocab, fp32 logits, row-major, ld = V). Histories are penalised whole
(repeat_last = 0), so an H-id history penalises every distinct id in it:
  single  1 x 49152  N(0, 2.5^2) + 8 ids spiked by +8; H=64; repeat 1.1, temp .7, top-k 40,
          top-p .9, min-p 0, seed 42; drawn 10,000 times on the same row.
  greedy  64 x 151936  N(0, 3^2); H=256 per row; repeat 1.15, temp 0; rows 0,10,20,.. hold a
          second index equal to the row's penalised maximum (an exact tie).
  peaked  256 x 151936  2*Gumbel(0,1) + 12*rank^-1.1 over a random 2,000-id permutation; H=512 with
          half the ids from the boosted set; repeat 1.1, temp .8, top-k 50, top-p .95,
          min-p .05, seeds 0..255 (one shared parameter block with seed 0: row r draws from
          the stream seeded with r).
  wide    512 x 151936  N(0, 0.5^2); top-k 0, top-p .99, min-p 0, temp 1, repeat 1.
  mixed   1024 x 128256  N(0, 2^2) + 1..16 spikes of +U[4,10] per row; per-row temp U[0,1.5]
          (25% exactly 0), top-k in {0,20,40,100}, top-p U[.8,1], min-p in {0,.05,.1},
          repeat U[1,1.3], H U[0,2048], seed = 1000 + row.
"""
import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

SAMPLING_DTYPE = np.dtype([("temp", "f4"), ("top_k", "i4"), ("top_p", "f4"), ("min_p", "f4"),
                           ("repeat", "f4"), ("repeat_last", "i4"), ("seed", "u8")])

WORKLOADS = ("single", "greedy", "peaked", "wide", "mixed")
SHAPES = {"single": (1, 49152), "greedy": (64, 151936), "peaked": (256, 151936), "wide": (512, 151936),
          "mixed": (1024, 128256)}
DATA_SEED = {"single": 0x51, "greedy": 0x52, "peaked": 0x53, "wide": 0x54, "mixed": 0x55}


def splitmix(seed, start, n):
    """Outputs start..start+n-1 of the SplitMix64 stream seeded with `seed` (uint64 array)."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def uniform(seed, start, n):
    """U(0,1) open interval, 53-bit."""
    return ((splitmix(seed, start, n) >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed, start, n):
    """N(0,1) in fp64 by Box-Muller over stream positions start..start+2n."""
    u = uniform(seed, 2 * start, 2 * n)
    u1, u2 = u[0::2], u[1::2]
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def gumbel(seed, start, n):
    return -np.log(-np.log(uniform(seed, start, n)))


def _ints(seed, start, n, lo, hi):
    """Integers uniform in [lo, hi)."""
    return lo + (splitmix(seed, start, n) % np.uint64(hi - lo)).astype(np.int64)


def _perm_prefix(seed, V, m):
    """First m entries of a seeded random permutation of range(V)."""
    keys = splitmix(seed, 0, V)
    return np.argsort(keys, kind="stable")[:m]


class Workload:
    """A materialised workload: logits [B,V] fp32, params (1 or B SAMPLING_DTYPE entries),
    CSR history (hist int32, hist_off int32 [B+1]) and per-row seeds."""

    def __init__(self, name, logits, params, hist, hist_off, draws=1):
        self.name = name
        self.logits = logits
        self.B, self.V = logits.shape
        self.params = params
        self.hist = hist
        self.hist_off = hist_off
        self.draws = draws

    @property
    def per_row(self):
        return self.params.size == self.B and self.B > 1

    def row_params(self, r):
        return self.params[r if self.per_row else 0]

    def h_eff(self):
        """Distinct in-range history ids that the penalty touches, per row (0 when it is off)."""
        out = np.zeros(self.B, dtype=np.int64)
        for r in range(self.B):
            p = self.row_params(r)
            if p["repeat"] == np.float32(1.0):
                continue
            h = self.hist[self.hist_off[r]:self.hist_off[r + 1]]
            rl = int(p["repeat_last"])
            if rl > 0 and h.size > rl:
                h = h[h.size - rl:]
            h = np.unique(h)
            out[r] = int(((h >= 0) & (h < self.V)).sum())
        return out

    def algorithmic_bytes(self):
        """Bytes a sampler must move per call: logits once, penalised history ids, output ids,
        per-row parameters when they are per row."""
        b = 4 * self.B * self.V + 4 * int(self.h_eff().sum()) + 4 * self.B
        if self.per_row:
            b += 32 * self.B
        return b


def _csr(lists):
    off = np.zeros(len(lists) + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(x) for x in lists])
    hist = np.concatenate([np.asarray(x, dtype=np.int32) for x in lists]) if off[-1] else np.zeros(0, np.int32)
    return hist.astype(np.int32), off


def _params(**kw):
    p = np.zeros(1, dtype=SAMPLING_DTYPE)
    for k, v in kw.items():
        p[k] = v
    return p


def make(name, rows=None):
    """Build workload `name`. `rows` (optional) keeps only the first `rows` rows (for quick tests)."""
    B, V = SHAPES[name]
    if rows is not None:
        B = min(B, rows)
    s = DATA_SEED[name]
    lg = np.empty((B, V), dtype=np.float32)
    if name == "single":
        x = 2.5 * normal(s, 0, V)
        spikes = _ints(s + 1, 0, 8, 0, V)
        x[spikes] += 8.0
        lg[0] = x.astype(np.float32)
        hist, off = _csr([_ints(s + 2, 0, 64, 0, V)])
        p = _params(temp=0.7, top_k=40, top_p=0.9, min_p=0.0, repeat=1.1, repeat_last=0, seed=42)
        return Workload(name, lg, p, hist, off, draws=10000)
    if name == "greedy":
        hl = []
        for r in range(B):
            lg[r] = (3.0 * normal(s, r * V, V)).astype(np.float32)
            hl.append(_ints(s + 1, r * 256, 256, 0, V))
        hist, off = _csr(hl)
        p = _params(temp=0.0, top_k=40, top_p=0.9, min_p=0.0, repeat=1.15, repeat_last=0, seed=0)
        rep = np.float32(1.15)
        for r in range(0, B, 10):
            h = np.unique(hl[r])
            pen = lg[r].copy()
            v = pen[h]
            pen[h] = np.where(v > 0, v / rep, v * rep).astype(np.float32)
            a = int(np.argmax(pen))
            mask = np.ones(V, bool)
            mask[h] = False
            mask[a] = False
            cands = np.flatnonzero(mask)
            j = int(cands[int(_ints(s + 2, r, 1, 0, cands.size)[0])])
            lg[r, j] = pen[a]
        return Workload(name, lg, p, hist, off)
    if name == "peaked":
        hl = []
        for r in range(B):
            boost = _perm_prefix(s * 1000003 + r, V, 2000)
            x = 2.0 * gumbel(s, r * V, V)
            x[boost] += 12.0 * np.arange(1, 2001, dtype=np.float64) ** -1.1
            lg[r] = x.astype(np.float32)
            nb = 256
            h = np.concatenate([boost[_ints(s + 1, r * 512, nb, 0, 2000)], _ints(s + 2, r * 512, 512 - nb, 0, V)])
            hl.append(h)
        hist, off = _csr(hl)
        # one shared parameter block: with seed 0, row r's draw stream is seeded with r
        p = _params(temp=0.8, top_k=50, top_p=0.95, min_p=0.05, repeat=1.1, repeat_last=0, seed=0)
        return Workload(name, lg, p, hist, off)
    if name == "wide":
        for r in range(B):
            lg[r] = (0.5 * normal(s, r * V, V)).astype(np.float32)
        hist, off = _csr([[] for _ in range(B)])
        p = _params(temp=1.0, top_k=0, top_p=0.99, min_p=0.0, repeat=1.0, repeat_last=0, seed=7)
        return Workload(name, lg, p, hist, off)
    if name == "mixed":
        hl = []
        p = np.zeros(B, dtype=SAMPLING_DTYPE)
        u = uniform(s + 3, 0, 8 * B).reshape(B, 8)
        for r in range(B):
            x = 2.0 * normal(s, r * V, V)
            ns = 1 + int(u[r, 0] * 16)
            sp = _ints(s + 1, r * 16, ns, 0, V)
            x[sp] += 4.0 + 6.0 * uniform(s + 2, r * 16, ns)
            lg[r] = x.astype(np.float32)
            H = int(u[r, 1] * 2049)
            hl.append(_ints(s + 4, r * 2048, H, 0, V))
            p[r]["temp"] = 0.0 if u[r, 2] < 0.25 else 1.5 * u[r, 3]
            p[r]["top_k"] = (0, 20, 40, 100)[int(u[r, 4] * 4)]
            p[r]["top_p"] = 0.8 + 0.2 * u[r, 5]
            p[r]["min_p"] = (0.0, 0.05, 0.1)[int(u[r, 6] * 3)]
            p[r]["repeat"] = 1.0 + 0.3 * u[r, 7]
            p[r]["repeat_last"] = 0
            p[r]["seed"] = 1000 + r
        hist, off = _csr(hl)
        return Workload(name, lg, p, hist, off)
    raise ValueError(f"unknown workload {name!r}; one of {WORKLOADS}")


class DecodeCase:
    """A seeded multi-sequence decode: n sequences over a vocabulary of V, each with its own
    sampling options (the fields of verbo_gen_opts plus repeat_last), a prompt, and next-position
    logits that depend on the sequence, the step and the sequence's last id (so a different pick
    changes what follows). Id 0 is the stop id; from step stop_after[r] on it gets a large bonus
    in row r, so most sequences end on it, the others on max_tokens."""

    def __init__(self, n=24, V=4096, seed=0x60):
        self.n, self.V, self.seed = n, V, seed
        u = uniform(seed, 0, 8 * n).reshape(n, 8)
        self.opts = []
        self.repeat_last = []
        self.prompts = []
        self.stop_after = []
        for r in range(n):
            self.opts.append(dict(max_tokens=8 + int(u[r, 0] * 33),
                                  temp=(0.0, 0.5, 0.8, 1.2)[int(u[r, 1] * 4)],
                                  top_k=(0, 20, 40, 300)[int(u[r, 2] * 4)],
                                  top_p=(0.8, 0.95, 1.0)[int(u[r, 3] * 3)],
                                  min_p=(0.0, 0.05)[int(u[r, 4] * 2)],
                                  repeat=(1.0, 1.15, 1.3)[int(u[r, 5] * 3)],
                                  seed=100 + r))
            self.repeat_last.append((4, 16, 64)[r % 3])
            self.prompts.append(_ints(seed + 1, r * 64, int(u[r, 6] * 31), 1, V).astype(np.int32))
            self.stop_after.append(6 + int(u[r, 7] * 40))
        self.stop_ids = (0,)

    def logits(self, step, last):
        """Logits [n, V] (fp32) of every sequence's next position at `step`; last[r]: row r's last
        id (-1 before its first pick)."""
        x = np.empty((self.n, self.V), np.float32)
        for r in range(self.n):
            v = 2.0 * normal(self.seed + 2 + r, step * self.V, self.V)
            if last[r] >= 0:
                v[(int(last[r]) * 7 + 13) % self.V] += 3.0
            if step >= self.stop_after[r]:
                v[0] += 6.0
            x[r] = v.astype(np.float32)
        return x


class ServeCase:
    """A seeded request stream for a continuous-batching server: R requests arriving over time at a
    batched decoder of `slots` slots (fewer than R, so finished sequences' slots are taken again).
    Each request has the fields of verbo_gen_opts plus repeat_last, a prompt and an arrival step;
    its next-position logits depend only on the request, its own step (steps since it was
    admitted) and its last id, so a request decodes the same whatever else shares the batch. Id 0
    is the stop id; from its own step stop_after[j] on it gets a large bonus. A few requests ask for
    no tokens at all, and bursts arrive together, so some wait in the queue for a free slot."""

    def __init__(self, n=40, slots=8, V=4096, seed=0x70):
        self.n, self.slots, self.V, self.seed = n, slots, V, seed
        u = uniform(seed, 0, 10 * n).reshape(n, 10)
        self.opts, self.repeat_last, self.prompts, self.stop_after, self.arrival = [], [], [], [], []
        for j in range(n):
            mt = 4 + int(u[j, 0] * 30)
            if j % 13 == 5:
                mt = 0  # asks for nothing: finishes at once, takes no slot
            self.opts.append(dict(max_tokens=mt,
                                  temp=(0.0, 0.5, 0.8, 1.2)[int(u[j, 1] * 4)],
                                  top_k=(0, 20, 40, 300)[int(u[j, 2] * 4)],
                                  top_p=(0.8, 0.95, 1.0)[int(u[j, 3] * 3)],
                                  min_p=(0.0, 0.05)[int(u[j, 4] * 2)],
                                  repeat=(1.0, 1.15, 1.3)[int(u[j, 5] * 3)],
                                  seed=500 + j))
            self.repeat_last.append((4, 16, 64)[j % 3])
            self.prompts.append(_ints(seed + 1, j * 64, 1 + int(u[j, 6] * 40), 1, V).astype(np.int32))
            self.stop_after.append(3 + int(u[j, 7] * 30))
            # bursts: a third of the requests arrive at step 0, the others spread over 60 steps
            self.arrival.append(0 if u[j, 8] < 1 / 3 else int(u[j, 9] * 60))
        self.stop_ids = (0,)

    def logits(self, reqs, steps, last):
        """Logits [len(reqs), V] (fp32): row i is request reqs[i]'s next position at its own step
        steps[i], after its last id last[i] (-1 before its first pick)."""
        x = np.empty((len(reqs), self.V), np.float32)
        for i, (j, t, l) in enumerate(zip(reqs, steps, last)):
            v = 2.0 * normal(self.seed + 2 + j, int(t) * self.V, self.V)
            if l >= 0:
                v[(int(l) * 7 + 13) % self.V] += 3.0
            if t >= self.stop_after[j]:
                v[0] += 6.0
            x[i] = v.astype(np.float32)
        return x
