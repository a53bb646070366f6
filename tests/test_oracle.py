"""Pins of the CPU oracle (runs without a GPU).

Each check is chosen so a plausible mistake in the oracle fails it:
  - Philox4x32-10 against the published known-answer vectors (Random123 /
    Salmon et al. SC'11); xorshift32 against Marsaglia's published value.
  - get_pseudo_random against the reference's own src/data.c, compiled from
    its source into oracle/_ref/ (and against committed golden values).
  - exp / prob against fp64 libm (ulp bound) and monotone over every binary32
    input in [-104, 0].
  - The exact integer predicates (top-p need, draw target, fixed point) against
    Python big-integer / Fraction arithmetic.
  - O1's selection against a brute force written from the definitions (tiny
    rows, every parameter mix), and against invariants on larger rows.
  - O1 against O3 (restated sampler_ref, the reference's own oracle) under the
    reference's own acceptance rule (exact, or u*Z within 5e-4*Z of the
    token's CDF interval; src/validation.c:5075-5081).
  - Greedy one-stage against the reference's two-stage argmax structure.
  - Scoring (mode 2): the binary64 log against libm (ulp bound, powers of two,
    the range-reduction boundary), the NLL against an fp64 log-sum-exp, the
    exact fixed-point mass against an fp64 sum, and the special rows.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle as O
from pumice_amd import workloads as WL

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# --------------------------------------------------------------------------
# RNGs and the reference's input generator
# --------------------------------------------------------------------------

def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds
    assert O.philox4x32_10([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert O.philox4x32_10([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert O.philox4x32_10([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == [
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def _xorshift_py(x):
    x ^= (x << 13) & 0xFFFFFFFF
    x ^= x >> 17
    x ^= (x << 5) & 0xFFFFFFFF
    return x


def test_xorshift32_known_answers():
    # Marsaglia 2003, "Xorshift RNGs": seed 2463534242 -> 723471715 with (13, 17, 5)
    assert O.xorshift32(2463534242) == 723471715
    assert O.xorshift32(1) == 270369
    rng = np.random.default_rng(0)
    for x in rng.integers(1, 2**32, 200):
        assert O.xorshift32(int(x)) == _xorshift_py(int(x))


def test_get_pseudo_random_against_reference_data_c():
    ref = O.ref_data_lib()
    if ref is None:
        pytest.skip("oracle/_ref/libref_data.so not built (no reference checkout)")
    rng = np.random.default_rng(1)
    for _ in range(2000):
        i, j = int(rng.integers(0, 64)), int(rng.integers(0, 300000))
        seed = int(rng.integers(0, 2**31 - 1))
        a = np.float32(O.lib().oracle_get_pseudo_random(i, j, seed))
        b = np.float32(ref.get_pseudo_random(i, j, seed))
        assert a.view(np.uint32) == b.view(np.uint32), (i, j, seed)


def test_get_data_golden():
    with open(os.path.join(GOLDEN, "get_data_777001.json")) as f:
        g = json.load(f)
    x = O.get_data(777001, 1, WL.V_PRUNED)[0]
    for j, bits in zip(g["ids"], g["bits"]):
        assert int(x[j].view(np.uint32)) == bits


# --------------------------------------------------------------------------
# exp / prob
# --------------------------------------------------------------------------

def _ulp(y):
    y = abs(float(y))
    if y < 2.0**-126:
        return 2.0**-149
    return 2.0 ** (math.frexp(y)[1] - 24)


def test_exp_monotone_exhaustive_and_accurate():
    viol, max_ulp, worst = O.exp_scan(-104.0, 0.0, 4096)
    assert viol == 0, f"pss_exp not monotone: {viol} violations"
    assert max_ulp <= 1.1, f"pss_exp error {max_ulp} ulp at {worst}"


def test_exp_special_points():
    x = np.array([0.0, -0.0, -1.0, -87.3, -103.9, -104.0, -104.5, -np.inf, -150.0], np.float32)
    y = O.exp_many(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[7] == 0.0 and y[8] == 0.0 and y[6] == 0.0
    ref = np.exp(x.astype(np.float64))
    for a, b in zip(y[2:5], ref[2:5]):
        assert abs(float(a) - b) <= 1.1 * _ulp(b)
    assert 0 < y[3] < 2.0**-126 or y[3] > 0  # subnormal range is produced, not flushed


def test_prob_accuracy_and_monotone():
    rng = np.random.default_rng(2)
    for tmax in [0.0, 0.5, 17.3, -5.0, 60.0, 1000.0, 3.0e6]:
        # dense: 2^20 consecutive floats below tmax
        start = np.float32(tmax).view(np.int32)
        if tmax > 0:
            bits = start - np.arange(1 << 20, dtype=np.int32)
        else:
            bits = (np.float32(tmax) if tmax != 0 else np.float32(-0.0)).view(np.int32) + np.arange(1 << 20, dtype=np.int32)
        t = bits.view(np.float32)
        t = t[np.isfinite(t) & (t <= np.float32(tmax))]
        p = O.prob_many(t, tmax)
        assert np.all(np.diff(p.astype(np.float64)) <= 0), f"prob not monotone below tmax={tmax}"
        # wide: random t over [tmax - 104, tmax]
        tw = (np.float32(tmax) - rng.uniform(0, 104, 200000).astype(np.float32)).astype(np.float32)
        pw = O.prob_many(tw, tmax).astype(np.float64)
        ref = np.exp(tw.astype(np.float64) - np.float64(np.float32(tmax)))
        ok = ref > 1e-37
        rel = np.abs(pw[ok] - ref[ok]) / ref[ok]
        assert rel.max() < 1.2e-7, f"prob rel err {rel.max()} at tmax={tmax}"
    assert O.prob_many(np.array([np.inf], np.float32), np.inf)[0] == 1.0
    assert O.prob_many(np.array([-np.inf], np.float32), -np.inf)[0] == 1.0
    assert O.prob_many(np.array([1.0], np.float32), np.inf)[0] == 0.0


# --------------------------------------------------------------------------
# exact integer predicates
# --------------------------------------------------------------------------

def test_topp_need_exact():
    rng = np.random.default_rng(3)
    tops = list(rng.uniform(0, 1, 300).astype(np.float32)) + [np.float32(1e-30), np.float32(1e-44),
                                                            np.float32(0.5), np.nextafter(np.float32(1), np.float32(0))]
    zks = [1, 2**45, 2**45 + 12345, 2**62 + 7, 2**63 - 1, 3]
    for tp in tops:
        if not (0 < tp < 1):
            continue
        for zk in zks + [int(v) for v in rng.integers(1, 2**63, 5, dtype=np.uint64)]:
            exact = Fraction(float(tp)) * zk
            need = math.ceil(exact)
            assert O.topp_need(float(tp), zk) == need, (float(tp), zk)


def test_draw_target_exact():
    rng = np.random.default_rng(4)
    for _ in range(3000):
        u = int(rng.integers(0, 2**24))
        z = int(rng.integers(1, 2**63, dtype=np.uint64))
        assert O.draw_target(u, z) == (u * z) >> 24
    assert O.draw_target(2**24 - 1, 2**63 - 1) == ((2**24 - 1) * (2**63 - 1)) >> 24


def test_fixq_and_keys():
    rng = np.random.default_rng(5)
    p = np.concatenate([rng.uniform(0, 1, 1000), [0.0, 1.0, 1e-45, 2.0**-45, 2.0**-46]]).astype(np.float32)
    for v in p:
        assert O.fixq(float(v)) == math.floor(Fraction(float(v)) * 2**45)
    t = np.concatenate([rng.standard_normal(4000) * 10, [0.0, np.inf, -np.inf, 1e-40, -1e-40]]).astype(np.float32)
    k = O.keys(t)
    order_t = np.argsort(t, kind="stable")
    assert np.all(np.diff(k[order_t].astype(np.int64)) >= 0)
    for v in t[:50]:
        assert np.float32(O.lib().oracle_unkey(O.key(float(v)))).view(np.uint32) == v.view(np.uint32)
    assert O.lib().oracle_canon(-0.0) == 0.0 and math.copysign(1, O.lib().oracle_canon(-0.0)) == 1.0
    assert O.lib().oracle_canon(float("nan")) == -math.inf


# --------------------------------------------------------------------------
# O1 selection vs a brute force from the definitions
# --------------------------------------------------------------------------

def brute_force(x, prm, hist, pos, rng_state, row=0, rng_mode=0):
    """Definitions, evaluated independently of O1: fp32 transform with numpy,
    probabilities from pss_prob (pinned above), exact rationals for masses."""
    T = np.float32(prm["temperature"])
    V = x.size
    if not (T > 0):
        k = O.keys(np.where(np.isnan(x), -np.inf, x + np.float32(0)).astype(np.float32))
        return int(np.argmax(k)), None
    W = min(int(prm["penaltyLength"]), 1024)
    with np.errstate(all="ignore"):
        invT = np.float32(1) / T
        pres = np.float32(prm["presencePenalty"]) * invT
        rep = np.float32(prm["repPenalty"])
        t = (x * invT).astype(np.float32)
        if W > 0 and (rep != 1 or pres != 0):
            ids = {int(h) for h in hist[:W] if h < V}
            for j in ids:
                v = t[j]
                if rep != 1:
                    v = np.float32(v / rep) if v > 0 else np.float32(v * rep)
                t[j] = np.float32(v - pres)
        t = np.where(np.isnan(t), np.float32(-np.inf), t + np.float32(0)).astype(np.float32)
    k = O.keys(t)
    tmax = t[np.argmax(k)]
    p = O.prob_many(t, tmax)
    q = [math.floor(Fraction(float(v)) * 2**45) for v in p]
    K = min(int(prm["topK"]), V)
    vals = sorted(set(int(v) for v in k), reverse=True)
    tau = 0
    if K > 0:
        tau = int(np.sort(k)[::-1][K - 1])
    zk = sum(q[j] for j in range(V) if k[j] >= tau)
    tp = float(np.float32(prm["topP"]))
    if 0 < tp < 1:
        need = Fraction(tp) * zk
        cands = [v for v in vals if v >= tau and sum(q[j] for j in range(V) if k[j] >= v) >= need]
        tau = max(tau, max(cands))
    mp = float(np.float32(prm["minP"]))
    kept = [bool(k[j] >= tau and (mp <= 0 or p[j] >= np.float32(mp))) for j in range(V)]
    z = sum(q[j] for j in range(V) if kept[j])
    if rng_mode == 0:
        s = rng_state if rng_state else 0x9E3779B9
        u24 = s >> 8
    else:
        u24 = O.philox4x32_10([0, row, 0, 0], [rng_state, 0])[0] >> 8
    cum = 0
    for j in range(V):
        if kept[j]:
            cum += q[j]
            if Fraction(cum) > Fraction(u24, 2**24) * z:
                return j, dict(kept=kept, z=z, tau=tau, zk=zk)
    raise AssertionError("no token crossed the target")


def test_o1_matches_brute_force():
    rng = np.random.default_rng(6)
    n = 0
    for trial in range(250):
        V = int(rng.integers(1, 40))
        if trial % 3 == 0:
            x = rng.integers(-3, 3, V).astype(np.float32)          # heavy ties
        else:
            x = (rng.standard_normal(V) * rng.uniform(0.1, 8)).astype(np.float32)
        prm = O.make_params(
            temperature=float(rng.choice([0.0, 0.3, 0.7, 1.0, 2.5])),
            repPenalty=float(rng.choice([1.0, 0.7, 1.3])),
            penaltyLength=int(rng.choice([0, 3, 10])),
            topK=int(rng.choice([0, 1, 2, 5, 50])),
            topP=float(rng.choice([1.0, 0.2, 0.5, 0.9, 0.0])),
            minP=float(rng.choice([0.0, 0.05, 0.3, 1.0])),
            presencePenalty=float(rng.choice([0.0, 0.5, -0.4])),
        )[0]
        hist = O.new_history()
        hist[:10] = rng.integers(0, V + 3, 10)
        seed = int(rng.integers(0, 2**32))
        for rng_mode in (0, 1):
            st = O.RowState(hist, 0, seed, 0)
            o = O.o1_row(x, prm, st, rng_mode=rng_mode)
            tok, extra = brute_force(x, prm, hist, 0, seed, 0, rng_mode)
            assert o["token"] == tok, (trial, rng_mode, V, prm)
            if extra is not None:
                assert [bool(v) for v in o["kept"]] == extra["kept"], trial
                assert int(o["info"]["z_kept"]) == extra["z"]
                assert int(o["info"]["tau_key"]) == extra["tau"]
                assert int(o["info"]["z_topk"]) == extra["zk"]
            n += 1
    assert n == 500


def test_o1_invariants_large_rows():
    rng = np.random.default_rng(7)
    V = 20000
    for trial in range(12):
        x = (rng.standard_normal(V) * 3).astype(np.float32)
        if trial % 4 == 1:
            x = np.round(x).astype(np.float32)
        K = int(rng.choice([0, 1, 40, 1000]))
        tp = float(rng.choice([1.0, 0.9, 0.5]))
        mp = float(rng.choice([0.0, 0.05]))
        prm = O.make_params(temperature=0.8, topK=K, topP=tp, minP=mp)[0]
        st = O.RowState(None, 0, int(rng.integers(1, 2**32)), 0)
        o = O.o1_row(x, prm, st, want_p=True)
        kept = o["kept"].astype(bool)
        t = (x * np.float32(1 / np.float32(0.8))).astype(np.float32)
        t = (x * (np.float32(1) / np.float32(0.8))).astype(np.float32)
        assert kept[o["token"]]
        assert kept[np.argmax(t)]
        # up-set in t: every kept value >= every dropped value's ... no dropped value above a kept one
        if kept.all():
            continue
        assert t[kept].min() >= t[~kept].max() or mp > 0
        if K and tp >= 1 and mp == 0:
            assert kept.sum() >= min(K, V)
            kth = np.sort(t)[::-1][K - 1]
            assert np.array_equal(kept, t >= kth)


# --------------------------------------------------------------------------
# O1 vs the reference's own oracle (O3) and the shader restatement (O2)
# --------------------------------------------------------------------------

def _accepts(x, prm, hist, pos, rng_state, tok):
    """O3 (sampler_ref) acceptance: exact, or within 5e-4 * Z of tok's interval."""
    h = hist.copy()
    t3, tol, _, _, _ = O.o3_sampler_ref(x, prm, h, pos, rng_state, accept_tok=tok, tol=5e-4)
    return t3 == tok, tol


def test_o1_accepted_by_reference_oracle_on_validator_cases():
    V = WL.V_PRUNED
    hist, pos0, cases, seeds = WL.validator_inputs(V)
    x = O.get_data(777001, 1, V)[0]
    st = O.RowState(hist, pos0, 0, 0)
    for c in range(4):
        st.rng = int(seeds[c])
        for d in range(3):
            h_before, pos_before, rng_before = st.history.copy(), st.position, st.rng
            o = O.o1_row(x, cases[c], st, want_p=True)
            ok, tol = _accepts(x, cases[c], h_before, pos_before, rng_before, o["token"])
            assert ok, f"case {'ABCD'[c]} draw {d}: O1 token {o['token']} rejected by sampler_ref"
            x = o["p"]


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_o1_accepted_by_reference_oracle_on_configs(name):
    if name == "c2":
        w, _ = WL.c2(seed=11, rows=16)
    elif name == "c3":
        w = WL.c3(seed=12, rows=16)
    else:
        w = WL.c4(seed=13, rows=4)
    exact = 0
    for r in range(w.rows):
        x = w.logits[r].astype(np.float32)
        st = O.RowState(w.history[r], 0, int(w.seeds[r]), 0)
        o = O.o1_row(x, w.params[r], st)
        ok, tol = _accepts(x, w.params[r], w.history[r], 0, int(w.seeds[r]), o["token"])
        assert ok, f"{name} row {r}"
        exact += not tol
    assert exact >= w.rows - 1


def test_shader_restatement_agreement_rate():
    """O2 (the reference shader's bisection, restated) against O1: the token
    agrees on most draws; disagreements are the reference's own bisection /
    fp32 boundary effects and stay within sampler_ref's acceptance."""
    w, xs = WL.c2(seed=14, rows=1, steps=40)
    agree = 0
    for k in range(40):
        x = xs[k, 0]
        st = O.RowState(w.history[0], 0, 1000 + k, 0)
        o1 = O.o1_row(x, w.params[0], st)
        h = w.history[0].copy()
        t2, _, _, _, _ = O.o2_shader_row(x, w.params[0], h, 0, 1000 + k)
        agree += (t2 == o1["token"])
        ok, _ = _accepts(x, w.params[0], w.history[0], 0, 1000 + k, t2)
        assert ok, f"step {k}: shader restatement token rejected by sampler_ref"
    assert agree >= 36


def test_greedy_one_stage_equals_two_stage():
    rng = np.random.default_rng(8)
    for trial in range(30):
        V = int(rng.choice([1, 255, 256, 257, 102400, 248320]))
        x = rng.integers(-5, 6, V).astype(np.float32) if trial % 2 else rng.standard_normal(V).astype(np.float32)
        if trial % 5 == 0:
            x[rng.integers(0, V, 3)] = np.float32(9.0)
        g1, g2 = O.greedy(x), O.greedy_two_stage(x)
        assert g1 == g2
        assert g1 == int(np.nonzero(x == x.max())[0][0])


def test_o1_batch_matches_rows_and_threads():
    w = WL.c3(seed=15, rows=8)
    hist = w.history.copy()
    pos = np.zeros(8, np.uint32)
    rng_s = w.seeds.copy()
    step = np.zeros(8, np.uint32)
    toks, infos = O.o1_batch(w.logits, w.params, hist, pos, rng_s, step, threads=3)
    for r in range(8):
        st = O.RowState(w.history[r], 0, int(w.seeds[r]), 0)
        o = O.o1_row(w.logits[r].astype(np.float32), w.params[r], st, row=r)
        assert o["token"] == int(toks[r])
        assert st.rng == int(rng_s[r]) and np.array_equal(st.history, hist[r])


# --------------------------------------------------------------------------
# committed golden fixtures (tests/golden/make_golden.py)
# --------------------------------------------------------------------------

def test_validator_golden():
    with open(os.path.join(GOLDEN, "validator_o1.json")) as f:
        g = json.load(f)
    V = g["V"]
    hist, pos0, cases, seeds = WL.validator_inputs(V)
    x = O.get_data(777001, 1, V)[0]
    st = O.RowState(hist, pos0, 0, 0)
    i = 0
    for c in range(4):
        st.rng = int(seeds[c])
        for d in range(3):
            o = O.o1_row(x, cases[c], st, want_p=True)
            exp = g["draws"][i]
            for f, v in exp["o1"].items():
                assert int(o["info"][f]) == v, (exp["case"], d, f)
            assert exp["o3_token"] == o["token"], "O1 and sampler_ref disagree on a validator draw"
            x = o["p"]
            i += 1
    assert st.position == g["final_position"]
    assert int(st.history.astype(np.uint64).sum()) == g["final_history_sum"]


def test_configs_golden():
    with open(os.path.join(GOLDEN, "configs_o1.json")) as f:
        g = json.load(f)
    w, _ = WL.c1(seed=0)
    assert O.greedy(w.logits[0]) == g["c1_greedy"]
    st = O.RowState(w.history[0], 0, 0, 0)
    assert O.o1_row(w.logits[0], w.params[0], st)["token"] == g["c1_sample"]
    w, xs = WL.c2(seed=24, rows=1, steps=8)
    st = O.RowState(w.history[0], 0, 99, 0)
    assert [O.o1_row(xs[k, 0], w.params[0], st)["token"] for k in range(8)] == g["c2_chain"]
    st = O.RowState(w.history[0], 0, 99, 0)
    assert [O.o1_row(xs[k, 0], w.params[0], st, rng_mode=1)["token"] for k in range(8)] == g["c2_chain_philox"]


def test_log64_against_libm():
    """pss_log64 (shared by the scoring kernel and the oracle): within 1 ulp of
    libm's log over 2^-20 .. 2^40, exact at powers of two, continuous across the
    sqrt(1/2) range-reduction boundary.  A wrong series term or ln2 split
    fails the ulp bound by orders of magnitude."""
    rng = np.random.default_rng(5)
    xs = np.concatenate([np.exp2(rng.uniform(-20, 40, 20000)), 1.0 + rng.uniform(-1e-3, 1e-3, 2000),
                         [1.0, 2.0, 0.5, 3.0, 10.0, 262144.0, 2.0 ** 18 - 1, math.sqrt(0.5), math.sqrt(2.0)]])
    worst = 0.0
    for x in xs:
        x = float(x)
        got, ref = O.log64(x), math.log(x)
        if ref == 0.0:
            assert got == 0.0
            continue
        worst = max(worst, abs(got - ref) / math.ulp(ref))
    assert worst <= 1.0, worst
    for e in range(-30, 31):
        assert O.log64(2.0 ** e) == e * math.log(2.0) or abs(O.log64(2.0 ** e) - e * math.log(2.0)) <= math.ulp(e * math.log(2.0))
    b = math.sqrt(0.5)
    lo, hi = np.nextafter(b, 0.0), np.nextafter(b, 1.0)
    assert O.log64(float(lo)) < O.log64(b) <= O.log64(float(hi))


def _nll64(x, target):
    x = x.astype(np.float64)
    m = x.max()
    lt = x[target] if target < x.size else 0.0
    return math.log(np.exp(x - m).sum()) + m - lt


def test_score_oracle_against_fp64():
    """O1 scoring = log(Z) + gmax - l[target] within fp32 rounding of an fp64
    log-sum-exp; Zq * 2^-45 within binary32 rounding of the fp64 sum (each term
    is a binary32 exp, then truncated to 2^-45); gmax its key."""
    rng = np.random.default_rng(6)
    for V in (1, 7, 1000, 4096, 102400):
        for sigma in (0.5, 3.0, 20.0):
            x = (rng.normal(0.0, sigma, V)).astype(np.float32)
            for target in (0, V - 1, V // 2, V, V + 5):
                bits, zq, gk = O.o1_score_row(x, target)
                nll = float(np.uint32(bits).view(np.float32))
                ref = _nll64(x, target)
                assert abs(nll - ref) <= 2.0 * float(np.spacing(np.float32(abs(ref)))) + 1e-6 * abs(ref), (V, sigma, target)
                z64 = np.exp(x.astype(np.float64) - float(x.max())).sum()
                assert abs(zq * 2.0 ** -45 - z64) <= 2.0 ** -23 * z64 + V * 2.0 ** -45
                assert gk == O.key(float(x.max()))


def test_score_oracle_special_rows():
    V = 64
    x = np.zeros(V, np.float32)
    bits, zq, _ = O.o1_score_row(x, 3)          # all equal: log V
    assert np.uint32(bits).view(np.float32) == np.float32(math.log(V))
    assert zq == V << 45
    y = np.full(V, -np.inf, np.float32)
    bits, _, _ = O.o1_score_row(y, 0)            # all -inf: -inf - (-inf)
    assert np.isnan(np.uint32(bits).view(np.float32))
    z = np.zeros(V, np.float32)
    z[5] = np.inf
    bits, zq, _ = O.o1_score_row(z, 6)           # +inf max, finite target
    assert np.uint32(bits).view(np.float32) == np.float32(np.inf) and zq == 1 << 45
    w = np.arange(V, dtype=np.float32)
    w[9] = np.nan                                # NaN is -inf: contributes nothing
    b1, _, _ = O.o1_score_row(w, 10)
    w2 = w.copy()
    w2[9] = -np.inf
    b2, _, _ = O.o1_score_row(w2, 10)
    assert b1 == b2
