"""GPU parity over seeded random configurations: each case draws a vocabulary
size, logit dtype, row count, logit distribution and per-row parameters
(temperature, top-k up to 1,024, top-p, min-p, repetition and presence
penalties over windows up to 1,024 ids), and runs two steps on every kernel
form against the oracle, with the same bar as the configuration tests:
token ids, row diagnostics, kept masks, per-row state bit-exact and
normalized probabilities within 1e-6 relative of an fp64 evaluation.  The
cases mix rows the streaming forms finish from their candidate lists with
rows they hand to the general algorithm (top-k off or above 256, long
windows, heavy ties) inside one launch."""
import numpy as np
import pytest

from pumice_amd import sampler as S
from test_gpu_parity import PATH_IDS, PATHS, run_both

pytestmark = pytest.mark.gpu

N_CASES = 40


def _logits(rng, rows, V, dtype):
    kind = rng.integers(0, 5)
    if kind == 0:      # normal, random scale
        x = rng.standard_normal((rows, V)) * rng.uniform(0.5, 6.0)
    elif kind == 1:    # Zipf-shaped: -a ln(rank) + noise, ranks permuted per row
        x = np.empty((rows, V))
        for r in range(rows):
            x[r] = -rng.uniform(0.5, 1.5) * np.log(rng.permutation(V) + 1.0) + rng.normal(0, 0.5, V)
    elif kind == 2:    # few distinct values: heavy ties
        x = rng.integers(0, rng.integers(2, 40), size=(rows, V)).astype(np.float64) * 0.25
    elif kind == 3:    # normal with spikes
        x = rng.standard_normal((rows, V)) * 2.0
        for r in range(rows):
            x[r, rng.integers(0, V, rng.integers(1, 12))] += rng.uniform(5, 50)
    else:              # normal with non-finite entries
        x = rng.standard_normal((rows, V)) * 3.0
        for r in range(rows):
            m = rng.integers(0, V, rng.integers(0, 20))
            x[r, m] = rng.choice([np.nan, np.inf, -np.inf], size=m.size)
    return x.astype(dtype)


def _params(rng, rows, V):
    p = S.make_params(rows)
    for r in range(rows):
        p[r]["temperature"] = 0.0 if rng.random() < 0.1 else rng.uniform(0.1, 2.0)
        u = rng.random()
        p[r]["topK"] = 0 if u < 0.15 else (rng.integers(1, 65) if u < 0.6 else
                                           rng.integers(65, 257) if u < 0.85 else rng.integers(257, 1025))
        p[r]["topP"] = 1.0 if rng.random() < 0.3 else rng.uniform(0.3, 1.0)
        p[r]["minP"] = 0.0 if rng.random() < 0.4 else rng.uniform(0.0, 0.3)
        p[r]["repPenalty"] = 1.0 if rng.random() < 0.3 else rng.uniform(0.5, 2.0)
        p[r]["presencePenalty"] = 0.0 if rng.random() < 0.4 else rng.uniform(-1.0, 1.0)
        u = rng.random()
        p[r]["penaltyLength"] = 0 if u < 0.2 else (rng.integers(1, 257) if u < 0.8 else rng.integers(257, 1025))
    return p


def make_case(seed):
    rng = np.random.default_rng(1000 + seed)
    V = int(rng.choice([257, 2048, 5003, 16384, 40000, 65536, 102400, 248320]))
    dtype = np.float16 if rng.random() < 0.3 else np.float32
    rows = int(rng.integers(1, 13))
    x0 = _logits(rng, rows, V, dtype)
    x1 = _logits(rng, rows, V, dtype)
    p = _params(rng, rows, V)
    # ids past the vocabulary and empty slots (0xFFFFFFFF) in the history
    hist = rng.integers(0, V + V // 8 + 1, size=(rows, 1024), dtype=np.uint32)
    for r in range(rows):
        if rng.random() < 0.3:
            hist[r, rng.integers(0, 1024):] = 0xFFFFFFFF
    seeds = rng.integers(0, 2**32, rows, dtype=np.uint32)
    pos = rng.integers(0, 5000, rows, dtype=np.uint32)
    rng_mode = S.RNG_PHILOX if rng.random() < 0.5 else S.RNG_XORSHIFT32
    return dict(x0=x0, x1=x1, p=p, hist=hist, seeds=seeds, pos=pos, rng_mode=rng_mode,
                desc=f"V={V} {np.dtype(dtype).name} rows={rows}")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_config(seed, flags):
    c = make_case(seed)
    print(f"random case {seed}: {c['desc']}", flush=True)
    run_both(c["x0"], c["p"], c["seeds"], c["hist"], c["pos"], flags=flags, steps=2,
             step_logits=[c["x0"], c["x1"]], rng_mode=c["rng_mode"], want_probs=True,
             where=f"random {seed} ({c['desc']})")
