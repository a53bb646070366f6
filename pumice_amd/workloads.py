"""Synthetic inputs of the sampler benchmark configurations (numpy, seeded).

Each generator returns host arrays: logits [rows, V] (float32 or float16),
params (sample_params records), seeds, histories [rows, 1024] and positions.
There is no dataset: logits are drawn from the distributions the benchmark
configurations name.

  c1  1 x 102,400 f32 ~ N(0, 2.5^2) + 8 ids set to +12 (an 8-way tie for
      greedy); then T 0.7 / top-k 40 / top-p 0.9, seed 0
  c2  1 x 102,400 f32 ~ N(0, 3^2) per step; rep 1.1, presence 0.5, window 64
      of ids uniform over the vocab; T 0.8, top-k 40, top-p 0.95, min-p 0.05
  c3  256 x 102,400 f16, logit = -1.1 ln(rank) + N(0, 0.5^2), ranks a random
      permutation per row; T ~ U[0.5, 1.2], top-k in {20, 40, 100},
      top-p ~ U[0.8, 1.0]; window 256, rep 1.1 (presence 0)
  c4  64 x 248,320 f32 ~ N(0, 3^2); top-k 1000, top-p 0.99, min-p 0.01,
      rep 1.05, window 512
  c5  128 x 102,400 f32 quantized to 16 values; some rows all equal, some
      rows with one id at +50; T 1, top-k 40, top-p 0.5, min-p 0.1
  headline  256 rows of c2 (f32, c2's sampler chain) -- the roofline case
"""
import numpy as np

V_PRUNED = 102400
V_FULL = 248320
MAX_PEN = 1024
SENTINEL = 0xFFFFFFFF

SAMPLE_PARAMS = np.dtype(
    [("temperature", "<f4"), ("repPenalty", "<f4"), ("penaltyLength", "<u4"), ("topK", "<u4"),
     ("topP", "<f4"), ("minP", "<f4"), ("presencePenalty", "<f4")]
)


def params(rows, temperature=1.0, repPenalty=1.0, penaltyLength=0, topK=0, topP=1.0, minP=0.0,
           presencePenalty=0.0):
    p = np.zeros(rows, SAMPLE_PARAMS)
    p["temperature"] = temperature
    p["repPenalty"] = repPenalty
    p["penaltyLength"] = penaltyLength
    p["topK"] = topK
    p["topP"] = topP
    p["minP"] = minP
    p["presencePenalty"] = presencePenalty
    return p


def histories(rng, rows, window, V):
    h = np.full((rows, MAX_PEN), SENTINEL, np.uint32)
    if window:
        h[:, :window] = rng.integers(0, V, size=(rows, window), dtype=np.uint32)
    return h


def normal_rows(rng, rows, V, sigma):
    return (rng.standard_normal((rows, V), dtype=np.float32) * np.float32(sigma)).astype(np.float32)


class Workload:
    def __init__(self, name, logits, params, seeds, history, position, dtype):
        self.name, self.logits, self.params = name, logits, params
        self.seeds, self.history, self.position, self.dtype = seeds, history, position, dtype

    @property
    def rows(self):
        return self.logits.shape[0]

    @property
    def V(self):
        return self.logits.shape[1]

    def bytes_per_row(self):
        """Algorithmic HBM bytes per sampled row: V*elem + 4*W + 44
        (history read, history write, params, rng, token, position)."""
        W = int(min(self.params["penaltyLength"].max(), MAX_PEN))
        return self.V * self.logits.dtype.itemsize + 4 * W + 44


def c1(seed=0, V=V_PRUNED):
    rng = np.random.default_rng(seed)
    x = normal_rows(rng, 1, V, 2.5)
    spikes = rng.choice(V, size=8, replace=False)
    x[0, spikes] = np.float32(12.0)
    p = params(1, temperature=0.7, topK=40, topP=0.9)
    return Workload("c1", x, p, np.zeros(1, np.uint32), histories(rng, 1, 0, V),
                    np.zeros(1, np.uint32), 0), np.sort(spikes)


def c2(seed=0, rows=1, V=V_PRUNED, steps=1):
    """`steps` fresh logit rows per state row: logits [steps, rows, V]."""
    rng = np.random.default_rng(seed)
    x = normal_rows(rng, steps * rows, V, 3.0).reshape(steps, rows, V)
    p = params(rows, temperature=0.8, repPenalty=1.1, penaltyLength=64, topK=40, topP=0.95,
               minP=0.05, presencePenalty=0.5)
    w = Workload("c2", x[0], p, np.zeros(rows, np.uint32), histories(rng, rows, 64, V),
                 np.zeros(rows, np.uint32), 0)
    return w, x


def headline(seed=0, rows=256, V=V_PRUNED):
    w, x = c2(seed, rows, V, 1)
    w.name = "headline"
    w.seeds = np.arange(rows, dtype=np.uint32)
    return w


def c3(seed=0, rows=256, V=V_PRUNED):
    rng = np.random.default_rng(seed)
    logr = np.log(np.arange(1, V + 1, dtype=np.float64))
    x = np.empty((rows, V), np.float16)
    for r in range(rows):
        ranks = rng.permutation(V)
        x[r] = (-1.1 * logr[ranks] + 0.5 * rng.standard_normal(V)).astype(np.float16)
    p = params(rows, repPenalty=1.1, penaltyLength=256)
    p["temperature"] = rng.uniform(0.5, 1.2, rows).astype(np.float32)
    p["topK"] = rng.choice(np.array([20, 40, 100], np.uint32), rows)
    p["topP"] = rng.uniform(0.8, 1.0, rows).astype(np.float32)
    return Workload("c3", x, p, rng.integers(1, 2**32, rows, dtype=np.uint32),
                    histories(rng, rows, 256, V), np.zeros(rows, np.uint32), 1)


def c4(seed=0, rows=64, V=V_FULL):
    rng = np.random.default_rng(seed)
    x = normal_rows(rng, rows, V, 3.0)
    p = params(rows, temperature=1.0, repPenalty=1.05, penaltyLength=512, topK=1000, topP=0.99,
               minP=0.01)
    return Workload("c4", x, p, rng.integers(1, 2**32, rows, dtype=np.uint32),
                    histories(rng, rows, 512, V), np.zeros(rows, np.uint32), 0)


def c5(seed=0, rows=128, V=V_PRUNED):
    rng = np.random.default_rng(seed)
    levels = np.sort(rng.normal(0.0, 3.0, 16)).astype(np.float32)
    # level index from a normal, so the top levels are rare but present
    idx = np.clip(np.round(rng.normal(7.5, 2.5, (rows, V))), 0, 15).astype(np.int64)
    x = levels[idx]
    kinds = np.arange(rows) % 8
    for r in np.nonzero(kinds == 1)[0]:        # all equal
        x[r, :] = levels[rng.integers(0, 16)]
    for r in np.nonzero(kinds == 2)[0]:        # one spike at +50
        x[r, rng.integers(0, V)] = np.float32(50.0)
    for r in np.nonzero(kinds == 3)[0]:        # only the top two levels
        x[r] = levels[14 + (rng.random(V) < 0.5)]
    p = params(rows, temperature=1.0, topK=40, topP=0.5, minP=0.1)
    return Workload("c5", x.astype(np.float32), p, rng.integers(1, 2**32, rows, dtype=np.uint32),
                    histories(rng, rows, 0, V), np.zeros(rows, np.uint32), 0)


def validator_inputs(V=V_PRUNED):
    """The reference validator's inputs (src/validation.c:5099-5120): logits
    getData(777001, 1, V) are computed by the oracle; this returns the history
    pattern, position, the four parameter cases A-D and their seeds."""
    hist = np.full(MAX_PEN, SENTINEL, np.uint32)
    for h in range(256):
        hist[h] = (h * 4099 + 17) % V
        if (h & 7) == 3:
            hist[h] = hist[h - 1]
        if (h & 31) == 5:
            hist[h] = SENTINEL
    cases = np.zeros(4, SAMPLE_PARAMS)
    cases[0] = (0.1, 1.2, 256, 40, 0.9, 0.0, 0.0)
    cases[1] = (0.1, 1.0, 0, 0, 1.0, 0.0, 0.0)
    cases[2] = (0.1, 1.0, 0, 0, 1.0, 0.001, 0.0)
    cases[3] = (0.1, 1.0, 256, 40, 0.9, 0.0, 0.3)
    seeds = np.array([0x2545F491, 0x9E3779B9, 0x85EBCA6B, 0x7F4A7C15], np.uint32)
    return hist, 7, cases, seeds
