"""GPU tests of the C generate-loop call site (pgl_generate, pgl_generate_pinned)
against a chain of O1 oracle steps: the prefill-final pass (no position
increment) and decode groups of four passes, emitted tokens of row 0, EOS and
the final per-row state (history ring, position, rng, Philox step) bit-exact."""
import numpy as np
import pytest

import oracle as O
from pumice_amd import generate as G
from pumice_amd import hip
from pumice_amd import sampler as S

pytestmark = pytest.mark.gpu

V = 4096
NBUF = 5
START = 3
SEED = 7


def _inputs(seed):
    rng = np.random.default_rng(seed)
    xs = rng.normal(0.0, 3.0, (NBUF, V)).astype(np.float32)
    params = O.make_params(temperature=0.8, repPenalty=1.1, presencePenalty=0.5, penaltyLength=16,
                           topK=40, topP=0.95, minP=0.05)
    hist = O.new_history()
    hist[:16] = rng.integers(0, V, 16, dtype=np.uint32)
    return xs, params, hist


def _oracle_chain(xs, params, hist, rng_mode, n):
    """Tokens of the prefill-final pass and n - 1 decode passes, and the state."""
    st = O.RowState(history=hist, position=START, rng=SEED, step=0)
    toks = [O.o1_row(xs[START % NBUF], params, st, rng_mode=rng_mode, do_increment=0,
                     want_kept=False)["token"]]
    for j in range(n - 1):
        toks.append(O.o1_row(xs[(START + j) % NBUF], params, st, rng_mode=rng_mode, do_increment=1,
                             want_kept=False)["token"])
    return toks, st


@pytest.mark.parametrize("pinned", [False, True], ids=["readback", "pinned"])
@pytest.mark.parametrize("rng_mode", [S.RNG_XORSHIFT32, S.RNG_PHILOX], ids=["xorshift", "philox"])
def test_generate_matches_oracle_chain(rng_mode, pinned):
    xs, params, hist = _inputs(21)
    max_new = 11  # prefill-final + groups of 4, 4, 2
    want, st = _oracle_chain(xs, params, hist, rng_mode, max_new)
    s = S.Sampler(V, 1)
    dev = [hip.DeviceBuffer.from_array(xs[k]) for k in range(NBUF)]
    pb = hip.PinnedBuffer(64) if pinned else None
    try:
        s.set_params(params, np.array([SEED], np.uint32))
        s.set_history(hist[None, :])
        table = G.LogitsTable([d.ptr for d in dev])
        toks, r = G.generate(s, table, max_new, rows=1, rng_mode=rng_mode, start_pos=START, pinned=pb)
        assert toks == want
        assert r["emitted"] == max_new and r["finish_reason"] == 1 and r["groups"] == 3
        got = s.read_state(1)
        assert np.array_equal(got["history"][0], st.history)
        assert int(got["position"][0]) == st.position == START + max_new - 1
        if rng_mode == S.RNG_XORSHIFT32:
            assert int(got["rng"][0]) == st.rng
        else:
            assert int(got["step"][0]) == st.step
    finally:
        s.close()
        for d in dev:
            d.free()
        if pb is not None:
            pb.free()


@pytest.mark.parametrize("pinned", [False, True], ids=["readback", "pinned"])
def test_generate_stops_at_eos(pinned):
    xs, params, hist = _inputs(22)
    want, _ = _oracle_chain(xs, params, hist, S.RNG_PHILOX, 9)
    eos = want[6]  # the sixth decode token (first occurrence decides)
    stop_at = want.index(eos) + 1
    s = S.Sampler(V, 1)
    dev = [hip.DeviceBuffer.from_array(xs[k]) for k in range(NBUF)]
    pb = hip.PinnedBuffer(64) if pinned else None
    try:
        s.set_params(params, np.array([SEED], np.uint32))
        s.set_history(hist[None, :])
        table = G.LogitsTable([d.ptr for d in dev])
        toks, r = G.generate(s, table, 50, rows=1, rng_mode=S.RNG_PHILOX, eos=eos, start_pos=START,
                             pinned=pb)
        assert toks == want[:stop_at]
        assert r["finish_reason"] == 0 and r["emitted"] == stop_at
    finally:
        s.close()
        for d in dev:
            d.free()
        if pb is not None:
            pb.free()
