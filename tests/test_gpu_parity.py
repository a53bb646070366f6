"""GPU parity: the HIP sampler through the C ABI against the O1 oracle, on the
benchmark configurations (reduced row counts so the oracle finishes in
seconds), the reference validator's cases, parameter edges, special values
and tiny / ragged vocabularies.  Bar: token ids, row diagnostics, kept masks,
probabilities and the per-row state (history ring, position, rng) bit-exact;
normalized probabilities within 1e-6 relative of an fp64 evaluation."""
import numpy as np
import pytest

import oracle as O
from harness import GpuRun, OracleRun, compare_state, compare_step
from pumice_amd import sampler as S
from pumice_amd import workloads as WL

pytestmark = pytest.mark.gpu

PATHS = [0, S.ENQ_FUSED, S.ENQ_SMALL, S.ENQ_SPLIT, S.ENQ_GENERAL, S.ENQ_RESIDENT]  # auto form, fused, small-batch, two-kernel, general, resident
PATH_IDS = ["auto", "fused", "small", "split", "general", "resident"]
PROB_RTOL = 1e-6                    # normalized probabilities vs fp64


def run_both(logits, params, seeds=None, history=None, position=None, flags=0, steps=1,
             step_logits=None, mode=S.MODE_SAMPLE, rng_mode=S.RNG_XORSHIFT32, do_increment=1,
             pass_idx=0, want_probs=False, where=""):
    g = GpuRun(logits, params, seeds, history, position)
    o = OracleRun(g.rows, params, seeds, history, position)
    try:
        for k in range(steps):
            x = logits if step_logits is None else step_logits[k]
            if step_logits is not None:
                g.load(x)
            go = g.step(mode, rng_mode, do_increment, pass_idx, want_mask=True,
                        want_probs=want_probs, flags=flags)
            oo = o.step(x, mode, rng_mode, do_increment, want_kept=True, want_probs=want_probs,
                        want_probs64=want_probs)
            compare_step(go, oo, pass_idx, check_probs=want_probs, where=f"{where} step {k}")
            if want_probs:
                for r in range(g.rows):
                    ref = oo[r]["probs64"]
                    got = go["probs"][r].astype(np.float64)
                    nz = ref > 0
                    rel = np.abs(got[nz] - ref[nz]) / ref[nz]
                    assert rel.max(initial=0.0) <= PROB_RTOL, f"{where} row {r}: prob rel err {rel.max()}"
                    assert np.all(got[~nz] == 0.0)
        compare_state(g.state(), o, where)
        return go
    finally:
        g.close()


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_c1_greedy_then_sample(flags):
    w, spikes = WL.c1(seed=0)
    g = run_both(w.logits, w.params, w.seeds, w.history, w.position, flags=flags,
                 mode=S.MODE_GREEDY, where="c1 greedy")
    if w.logits.max() == np.float32(12.0):
        assert int(g["tokens"][0]) == int(spikes[0]), "greedy must pick the smallest tied id"
    run_both(w.logits, w.params, w.seeds, w.history, w.position, flags=flags, want_probs=True,
             where="c1 sample")


@pytest.mark.parametrize("rng_mode", [S.RNG_XORSHIFT32, S.RNG_PHILOX], ids=["xorshift", "philox"])
@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_c2_chain(rng_mode, flags):
    w, x = WL.c2(seed=1, rows=1, steps=24)
    run_both(x[0], w.params, np.array([1234567], np.uint32), w.history, w.position, flags=flags,
             steps=24, step_logits=x, rng_mode=rng_mode, where="c2 chain")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_c2_probs(flags):
    w, x = WL.c2(seed=2, rows=2, steps=1)
    run_both(x[0], w.params, np.array([7, 0], np.uint32), w.history, w.position, flags=flags,
             want_probs=True, where="c2 probs")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_c3_fp16_zipf(flags):
    w = WL.c3(seed=3, rows=48)
    run_both(w.logits, w.params, w.seeds, w.history, w.position, flags=flags, where="c3")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_c4_unpruned(flags):
    w = WL.c4(seed=4, rows=6)
    run_both(w.logits, w.params, w.seeds, w.history, w.position, flags=flags, where="c4")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_c5_adversarial(flags):
    w = WL.c5(seed=5, rows=24)
    run_both(w.logits, w.params, w.seeds, w.history, w.position, flags=flags, want_probs=True,
             where="c5")


WIDE_CASES = {
    # name: (V, dtype, topK, W, window kind)
    "k300_w512_uniform": (102400, np.float32, 300, 512, "uniform"),
    "k1024_w1024_dups": (102400, np.float32, 1024, 1024, "dups"),
    "k700_w300_clustered": (248320, np.float32, 700, 300, "clustered"),
    "k257_w1024_f16": (65536, np.float16, 257, 1024, "uniform"),
    "k40_w600": (102400, np.float32, 40, 600, "uniform"),
    "k1000_small_vocab": (4000, np.float32, 1000, 64, "uniform"),
}


@pytest.mark.parametrize("flags", [0, S.ENQ_FUSED, S.ENQ_RESIDENT], ids=["auto", "fused", "resident"])
@pytest.mark.parametrize("case", sorted(WIDE_CASES))
def test_wide_fused(case, flags):
    """The wide fused form (top-k up to 1,024, windows up to 1,024 in LDS):
    duplicate window ids, ids at or beyond V, a window clustered in a few
    items, fp16, and a vocabulary too small for the joint certificate (the
    list then takes every element, or the row goes to the general algorithm);
    chained over two steps so the window ring advances."""
    V, dt, K, W, kind = WIDE_CASES[case]
    rng = np.random.default_rng(sum(case.encode()))
    rows = 5
    logits = rng.normal(0.0, 3.0, (rows, V)).astype(dt)
    params = O.make_params(temperature=0.9, repPenalty=1.2, presencePenalty=0.3, penaltyLength=W, topK=K,
                           topP=0.97, minP=0.01, rows=rows)
    hist = O.new_history(rows)
    for r in range(rows):
        if kind == "uniform":
            ids = rng.integers(0, V, W)
        elif kind == "dups":
            ids = rng.integers(0, 300, W)            # many duplicates
            ids[::7] = V + rng.integers(0, 5, ids[::7].size)  # ids beyond the vocab
        else:
            ids = rng.integers(0, 2048, W) + 4096 * (r + 1)   # one or two items
        hist[r, :W] = ids.astype(np.uint32)
    run_both(logits, params, np.arange(1, rows + 1, dtype=np.uint32), hist, None, flags=flags, steps=2,
             step_logits=[logits, np.roll(logits, 3, axis=1)], where=f"wide {case}")


@pytest.mark.parametrize("V", [248320, 248324, 131072, 65540])
def test_wide_split_mixed_rows(V):
    """The split-row wide form (auto choice for top-k above 256 or windows
    above 256 ids) on one launch mixing row kinds: top-k 1,000 / 300 / 1,024,
    top-k off (general algorithm in the finishing workgroup), greedy rows
    (temperature 0), no window, a row whose window repeats one id, a row of
    16 distinct values (bins of thousands of equal keys: the list finisher)
    and a row rounded to 1/64 (a few equal keys per bin: the histogram
    finisher's in-bin ranks); V with a partial last segment (248,324:
    51,716 ids in segment 3; 65,540: a second segment of 4 ids) or exact
    segments (131,072)."""
    rng = np.random.default_rng(V)
    rows = 10
    logits = rng.normal(0.0, 3.0, (rows, V)).astype(np.float32)
    logits[8] = np.sort(rng.normal(0.0, 3.0, 16)).astype(np.float32)[rng.integers(0, 16, V)]
    logits[9] = np.round(logits[9] * 64.0) / 64.0
    params = O.make_params(temperature=1.0, repPenalty=1.05, presencePenalty=0.2, penaltyLength=512, topK=1000,
                           topP=0.99, minP=0.01, rows=rows)
    params["topK"] = np.array([1000, 300, 1024, 0, 1000, 1000, 700, 1000, 1000, 900], np.uint32)
    params["temperature"][4] = 0.0
    params["penaltyLength"][5] = 0
    params["topP"][6] = 1.0
    params["minP"][7] = 0.0
    hist = O.new_history(rows)
    for r in range(rows):
        hist[r, :512] = rng.integers(0, V, 512).astype(np.uint32)
    hist[7, :512] = np.uint32(V - 1)
    run_both(logits, params, np.arange(1, rows + 1, dtype=np.uint32), hist, None, steps=2,
             step_logits=[logits, np.roll(logits, 5, axis=1)], where=f"wide split V={V}")


FULL_BATCHES = {
    # name: (generator, rows) -- row counts that select each fast-kernel shape
    "headline_256x102400_f32": (lambda: WL.headline(seed=31), None),   # 512 x 200, one segment
    "c3_256x102400_f16": (lambda: WL.c3(seed=32), None),               # 512 x 200, fp16
    "c5_128x102400_ties": (lambda: WL.c5(seed=33), None),              # 512 x 128, 2 segments
    "c4_64x248320": (lambda: WL.c4(seed=34), None),                    # 512 x 128, 4 segments
    "c2_120x65536": (lambda: WL.c2(seed=35, rows=120, V=65536)[0], None),  # 512 x 64, 2 segments
}


@pytest.mark.parametrize("name", sorted(FULL_BATCHES))
def test_full_batches(name):
    w = FULL_BATCHES[name][0]()
    seeds = w.seeds if w.seeds.any() else np.arange(w.rows, dtype=np.uint32) * 7919
    run_both(w.logits, w.params, seeds, w.history, w.position, steps=2,
             step_logits=[w.logits, np.roll(w.logits, 1, axis=1)], where=name)


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_reference_validator_cases(flags):
    """validateArgMaxSampler (src/validation.c:5094-5185): getData(777001) logits,
    the 256-slot history pattern, pos 7, cases A-D x 3 chained draws.  The
    reference chains draws through its in-place logits; here each draw's input
    is the previous draw's unnormalized p from O1, fed to both sides."""
    V = WL.V_PRUNED
    hist, pos0, cases, seeds = WL.validator_inputs(V)
    x = O.get_data(777001, 1, V)
    g = GpuRun(x, cases[:1], seeds[:1], hist[None, :], np.array([pos0], np.uint32))
    o = OracleRun(1, cases[:1], seeds[:1], hist[None, :], np.array([pos0], np.uint32))
    try:
        for c in range(4):
            g.s.set_params(cases[c:c + 1], seeds[c:c + 1])
            o.params = cases[c:c + 1].copy()
            o.states[0].rng, o.states[0].step = int(seeds[c]), 0
            for d in range(3):
                g.load(x)
                go = g.step(flags=flags)
                oo = o.step(x, want_p=True)
                compare_step(go, oo, where=f"case {'ABCD'[c]} draw {d}")
                x = oo[0]["p"][None, :].copy()
        st = g.state()
        compare_state(st, o, "validator")
        assert int(st["position"][0]) == pos0 + 12  # +1 per draw (doIncrement = 1)
    finally:
        g.close()


EDGE_PARAMS = [
    dict(temperature=1.0, topK=0),
    dict(temperature=1.0, topK=1),
    dict(temperature=1.0, topK=4099),
    dict(temperature=1.0, topK=100000),
    dict(temperature=0.5, topP=1e-30),
    dict(temperature=0.5, topP=0.0),
    dict(temperature=0.5, topP=0.5),
    dict(temperature=0.5, topP=1.5),
    dict(temperature=0.5, minP=1.0),
    dict(temperature=0.5, minP=-1.0),
    dict(temperature=0.5, minP=0.3, topK=7),
    dict(temperature=float("nan")),
    dict(temperature=-1.0),
    dict(temperature=0.0),
    dict(temperature=1e-30, topK=3),
    dict(temperature=1e-39, topK=3),
    dict(temperature=float("inf"), topK=10),
    dict(temperature=0.7, repPenalty=2.0, penaltyLength=40),
    dict(temperature=0.7, repPenalty=0.5, penaltyLength=40, topK=50),
    dict(temperature=0.7, presencePenalty=1.0, penaltyLength=40),
    dict(temperature=0.7, presencePenalty=-3.0, penaltyLength=40, topP=0.9),
    dict(temperature=0.7, repPenalty=1.3, presencePenalty=0.2, penaltyLength=2000, topK=20, topP=0.8, minP=0.02),
    dict(temperature=2.0, repPenalty=1.0, presencePenalty=0.0, penaltyLength=512, topK=5),
]


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_param_edges(flags):
    V = 4099
    rows = len(EDGE_PARAMS)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    x[:, ::97] = np.float32(1.5)   # some exact ties
    p = np.zeros(rows, S.SAMPLE_PARAMS)
    for r, kw in enumerate(EDGE_PARAMS):
        p[r] = tuple(S.make_params(1, **kw)[0])
    hist = np.full((rows, 1024), 0xFFFFFFFF, np.uint32)
    hist[:, :1024] = rng.integers(0, V + 50, size=(rows, 1024), dtype=np.uint32)
    seeds = rng.integers(0, 2**32, rows, dtype=np.uint32)
    seeds[0] = 0
    seeds[1] = 1
    run_both(x, p, seeds, hist, np.arange(rows, dtype=np.uint32) * 77, flags=flags, steps=3,
             step_logits=[x, x[::-1].copy(), -x], want_probs=True, where="edges")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_special_values(flags):
    V = 3000
    rng = np.random.default_rng(8)
    rows = 10
    x = rng.standard_normal((rows, V)).astype(np.float32)
    x[0, 5] = np.nan
    x[0, 9] = np.inf
    x[1, :] = -np.inf
    x[2, :] = np.nan
    x[3, 100] = np.inf
    x[3, 200] = np.inf
    x[4, ::2] = -0.0
    x[4, 1::2] = 0.0
    x[5, :] = np.float32(3.0)
    x[6, 17] = np.float32(3e38)
    x[6, 18] = np.float32(-3e38)
    x[7, :] = np.float32(1e-42)          # subnormal ties
    x[8, :100] = np.nan
    x[9, ::3] = -np.inf
    p = S.make_params(rows, temperature=0.9, topK=16, topP=0.9, minP=0.01)
    for mode in (S.MODE_SAMPLE, S.MODE_GREEDY):
        run_both(x, p, np.arange(rows, dtype=np.uint32), flags=flags, mode=mode,
                 want_probs=(mode == S.MODE_SAMPLE), where=f"special mode {mode}")


def _ulp_run(base, n, rng):
    """n binary32 values base, base + 1 ulp, ... in random order."""
    b = np.array([base], np.float32).view(np.uint32)[0]
    step = np.uint32(1) if base > 0 else np.uint32(0xFFFFFFFF)  # toward +inf
    v = (b + step * np.arange(n, dtype=np.uint32)).astype(np.uint32).view(np.float32)
    return rng.permutation(v)


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_rounding_ties(flags):
    """Rows whose K-th largest sits where t = l * (1/T) rounds distinct
    logits to one value (kernels that bound the K-th largest on l must
    still keep every tied t), where t overflows to +inf, and where t is
    subnormal; full-width rows so every kernel form takes them."""
    V = 102400
    rng = np.random.default_rng(21)
    rows = 6
    x = rng.standard_normal((rows, V)).astype(np.float32)
    T = [3.0, 7.0, 0.1, 1e-30, 1e38, 1.0 / 3.0]
    x[0, rng.choice(V, 300, replace=False)] = _ulp_run(np.float32(7.0), 300, rng)
    x[1, rng.choice(V, 300, replace=False)] = _ulp_run(np.float32(-0.03), 300, rng)
    x[1] -= np.float32(5.0)
    x[1, rng.choice(V, 300, replace=False)] = _ulp_run(np.float32(-0.03), 300, rng)
    x[2, rng.choice(V, 300, replace=False)] = _ulp_run(np.float32(7.0), 300, rng)
    x[3, rng.choice(V, 60, replace=False)] = np.float32(1e9) * (1 + rng.random(60, np.float32))
    x[4] *= np.float32(1e-3)
    x[5, rng.choice(V, 300, replace=False)] = _ulp_run(np.float32(1.5), 300, rng)
    p = S.make_params(rows, temperature=1.0, topK=40, topP=0.97, minP=0.0)
    p["temperature"] = np.array(T, np.float32)
    p[1]["topK"] = 150
    p[5]["topK"] = 200
    run_both(x, p, np.arange(rows, dtype=np.uint32) + 5, flags=flags, want_probs=True, where="rounding ties")
    xh = (rng.standard_normal((3, V)) * 4).astype(np.float16)
    xh[0, rng.choice(V, 100, replace=False)] = np.float16(60000.0)
    ph = S.make_params(3, temperature=1.0, topK=40, topP=0.97)
    ph["temperature"] = np.array([1e-35, 1e38, 0.37], np.float32)
    run_both(xh, ph, np.arange(3, dtype=np.uint32) + 9, flags=flags, where="rounding ties fp16")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_fp16_special(flags):
    V = 2048
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((4, V)) * 4).astype(np.float16)
    x[0, :64] = np.float16(6e-8)       # fp16 subnormals
    x[1, 7] = np.float16(np.inf)
    x[2, :] = np.float16(-65504.0)
    x[3, 3] = np.float16(np.nan)
    p = S.make_params(4, temperature=0.3, topK=50, topP=0.7)
    run_both(x, p, np.arange(4, dtype=np.uint32) + 11, flags=flags, where="fp16 special")


@pytest.mark.parametrize("V", [1, 2, 3, 31, 32, 33, 257, 1000])
@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_tiny_vocab(V, flags):
    rng = np.random.default_rng(V)
    rows = 6
    x = rng.standard_normal((rows, V)).astype(np.float32)
    p = S.make_params(rows, temperature=0.8, topK=3, topP=0.9, repPenalty=1.2, penaltyLength=4)
    p[1]["topK"] = 0
    p[2]["temperature"] = 0.0
    p[3]["minP"] = 0.5
    hist = np.full((rows, 1024), 0xFFFFFFFF, np.uint32)
    hist[:, :4] = rng.integers(0, V, size=(rows, 4), dtype=np.uint32)
    run_both(x, p, np.arange(rows, dtype=np.uint32), hist, flags=flags, steps=2,
             step_logits=[x, x * 0.5], want_probs=True, where=f"V={V}")


@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_slots_and_increment(flags):
    V = 5000
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, V)).astype(np.float32)
    p = S.make_params(3, temperature=1.0, topK=30, penaltyLength=3, repPenalty=1.5)
    g = GpuRun(x, p, np.array([3, 4, 5], np.uint32))
    o = OracleRun(3, p, np.array([3, 4, 5], np.uint32))
    try:
        for k, (slot, inc) in enumerate([(0, 1), (1, 0), (2, 1), (3, 1), (0, 0)]):
            go = g.step(pass_idx=slot, do_increment=inc, flags=flags)
            oo = o.step(x, do_increment=inc)
            compare_step(go, oo, pass_idx=slot, where=f"slot {slot}")
        compare_state(g.state(), o, "slots")
    finally:
        g.close()


def test_param_validation_errors():
    s = S.Sampler(100, 2)
    try:
        bad = [dict(topP=float("nan")), dict(minP=float("nan")), dict(repPenalty=float("nan")),
               dict(presencePenalty=float("nan")), dict(minP=1.5)]
        for kw in bad:
            with pytest.raises(S.PssError) as e:
                s.set_params(S.make_params(1, temperature=1.0, **kw))
            assert e.value.status == 1
        with pytest.raises(S.PssError):
            s.set_params(S.make_params(3))          # more rows than max_rows
        with pytest.raises(S.PssError):
            s.enqueue(0, 0, 100, 1)                 # null logits
        with pytest.raises(S.PssError):
            s.enqueue(1 << 20, 0, 99, 1)            # stride below vocab
        with pytest.raises(S.PssError):
            s.enqueue(1 << 20, 0, 100, 1, pass_idx=4)
        with pytest.raises(S.PssError):
            s.enqueue(1 << 20, 2, 100, 1)           # bad dtype
    finally:
        s.close()
    with pytest.raises(S.PssError) as e:
        S.Sampler(S.MAX_VOCAB + 1, 1)
    assert e.value.status == 4
