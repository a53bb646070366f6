"""GPU parity of the scoring mode (PSS_MODE_SCORE, ArgMax-Reduce.comp mode 2)
against the O1 scoring restatement: the result slot (float bits of the NLL,
NaN compared as NaN), token = target, position + do_increment, history / rng /
step untouched, and the row diagnostics (Zq, key of the maximum), over fp32 and
fp16 rows, tiny and ragged vocabularies, targets inside and outside the vocab,
every pass slot, and rows with NaN / +-inf."""
import numpy as np
import pytest

import oracle as O
from pumice_amd import hip
from pumice_amd import sampler as S

pytestmark = pytest.mark.gpu


def _same_bits(a, b):
    fa, fb = np.uint32(a).view(np.float32), np.uint32(b).view(np.float32)
    return (np.isnan(fa) and np.isnan(fb)) or int(a) == int(b)


def _run(x, targets, pass_idx=0, do_increment=1):
    """x [rows, V] (fp32 or fp16), targets [rows]; one scoring pass."""
    rows, V = x.shape
    dtype = S.DTYPE_F16 if x.dtype == np.float16 else S.DTYPE_F32
    s = S.Sampler(V, rows)
    dev = hip.DeviceBuffer.from_array(np.ascontiguousarray(x))
    info = hip.DeviceBuffer(rows * S.ROW_INFO.itemsize)
    try:
        s.set_params(O.make_params(temperature=0.8, repPenalty=1.1, penaltyLength=8, topK=40, rows=rows),
                     np.arange(1, rows + 1, dtype=np.uint32))
        hist = np.full((rows, 1024), 0xFFFFFFFF, np.uint32)
        hist[:, :8] = np.arange(8, dtype=np.uint32)
        s.set_history(hist)
        s.set_position(np.full(rows, 5, np.uint32))
        t = np.zeros((rows, 4), np.uint32)
        t[:, pass_idx] = targets
        s.set_score_targets(t)
        before = s.read_state(rows)
        s.enqueue(dev.ptr, dtype, V, rows, S.MODE_SCORE, do_increment, pass_idx, S.RNG_XORSHIFT32,
                  row_info=info.ptr)
        res, tok = s.read_results(rows)
        inf = info.download(S.ROW_INFO, rows)
        after = s.read_state(rows)
    finally:
        s.close()
        dev.free()
        info.free()
    for r in range(rows):
        want_bits, zq, gk = O.o1_score_row(x[r].astype(np.float32), int(targets[r]))
        got_bits = int(res[r][pass_idx])
        assert _same_bits(got_bits, want_bits), (r, hex(got_bits), hex(want_bits))
        assert int(tok[r]) == int(targets[r])
        assert int(inf[r]["z_kept"]) == zq and int(inf[r]["tmax_key"]) == gk
        assert int(inf[r]["flags"]) == S.INFO_SCORE
    assert np.array_equal(after["history"], before["history"])
    assert np.array_equal(after["rng"], before["rng"]) and np.array_equal(after["step"], before["step"])
    assert np.array_equal(after["position"], before["position"] + (1 if do_increment else 0))
    return res


@pytest.mark.parametrize("dtype", [np.float32, np.float16], ids=["f32", "f16"])
def test_score_batch(dtype):
    rng = np.random.default_rng(31)
    rows, V = 8, 102400
    x = rng.normal(0.0, 3.0, (rows, V)).astype(dtype)
    targets = rng.integers(0, V, rows).astype(np.uint32)
    targets[0] = int(np.argmax(x[0]))   # the row maximum itself
    targets[1] = V + 3                  # outside the vocab: scored against 0
    _run(x, targets)


@pytest.mark.parametrize("V", [1, 3, 33, 257, 1000, 4096])
def test_score_tiny_and_ragged_vocab(V):
    rng = np.random.default_rng(V)
    rows = 3
    x = rng.normal(0.0, 2.0, (rows, V)).astype(np.float32)
    targets = np.array([0, V - 1, V], np.uint32)
    _run(x, targets)


@pytest.mark.parametrize("pass_idx", [0, 1, 2, 3])
def test_score_slots_and_increment(pass_idx):
    rng = np.random.default_rng(40 + pass_idx)
    x = rng.normal(0.0, 3.0, (2, 5000)).astype(np.float32)
    _run(x, np.array([7, 4999], np.uint32), pass_idx=pass_idx, do_increment=pass_idx & 1)


def test_score_special_values():
    V = 2048
    x = np.random.default_rng(50).normal(0.0, 1.0, (6, V)).astype(np.float32)
    x[0, 100] = np.nan                  # NaN counts as -inf
    x[1, :] = -np.inf                   # all -inf: NaN result
    x[2, 17] = np.inf                   # +inf maximum
    x[3, :] = 0.0                       # all equal: log V
    x[4, 5] = -0.0
    x[5, 9] = np.inf
    x[5, 10] = np.inf                   # two +inf
    targets = np.array([100, 3, 17, 11, 5, 10], np.uint32)
    _run(x, targets)


def test_pgl_score_loop():
    """pgl_score (generateScore's consumption loop) over 11 ids: the sum of
    the per-pass NLLs (each bit-exact to O1) in id order, the count, and the
    position advanced once per id."""
    from pumice_amd import generate as G
    rng = np.random.default_rng(60)
    V, nbuf, start = 4096, 5, 2
    xs = rng.normal(0.0, 3.0, (nbuf, V)).astype(np.float32)
    ids = rng.integers(0, V, 11).astype(np.uint32)
    want = 0.0
    for j, t in enumerate(ids):
        bits, _, _ = O.o1_score_row(xs[(start + j) % nbuf], int(t))
        want += float(np.uint32(bits).view(np.float32))
    s = S.Sampler(V, 1)
    dev = [hip.DeviceBuffer.from_array(xs[k]) for k in range(nbuf)]
    try:
        table = G.LogitsTable([d.ptr for d in dev])
        loss, count = G.score(s, table, ids, start_pos=start)
        assert count == ids.size
        assert loss == want
        assert int(s.read_state(1)["position"][0]) == start + ids.size
    finally:
        s.close()
        for d in dev:
            d.free()
