import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden" / "sampler_golden.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.load_oracle()
    return O


@pytest.fixture(scope="session")
def golden():
    """The reference's picks (tests/golden/make_golden.py): list of case dicts."""
    import oracle as O
    from verbo_amd import workloads as W

    z = np.load(GOLDEN, allow_pickle=False)
    cases = []
    for i in range(int(z["n_cases"][0])):
        if f"case{i}_logits" in z:
            lg = z[f"case{i}_logits"]
        else:
            lg = np.full(int(z[f"case{i}_n"][0]), z[f"case{i}_fill"][0], np.float32)
        c = z[f"case{i}_cfg"][0]
        cases.append(dict(name=f"case{i}", logits=lg, cfg=O.Sampling(*[c[f].item() for f in O.SAMPLING_DTYPE.names]),
                          hist=z[f"case{i}_hist"], n=int(z[f"case{i}_run"][0]), accept=bool(z[f"case{i}_run"][1]),
                          ids=z[f"case{i}_ids"]))
    made = {}
    for j in range(int(z["n_wl"][0])):
        name = W.WORKLOADS[int(z[f"wl{j}_name"][0])]
        if name not in made:
            made[name] = W.make(name, rows=4)
        w = made[name]
        r = int(z[f"wl{j}_row"][0])
        c = z[f"wl{j}_cfg"][0]
        cases.append(dict(name=f"{name}[{r}]", logits=w.logits[r], sha=bytes(z[f"wl{j}_sha"]),
                          cfg=O.Sampling(*[c[f].item() for f in O.SAMPLING_DTYPE.names]),
                          hist=w.hist[w.hist_off[r]:w.hist_off[r + 1]], n=int(z[f"wl{j}_run"][0]),
                          accept=bool(z[f"wl{j}_run"][1]), ids=z[f"wl{j}_ids"]))
    return cases
