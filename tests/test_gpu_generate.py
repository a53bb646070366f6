"""GPU tests of the C generate-loop call site (pgl_generate, pgl_generate_pinned,
pgl_generate_pipelined) against a chain of O1 oracle steps: the prefill-final
pass (no position increment) and decode groups of four passes, emitted tokens
of row 0, EOS and the final per-row state (history ring, position, rng, Philox
step) bit-exact; the pipelined loop (next group queued before the current one
is read, PSS_ENQ_GATED passes) ends in the unpipelined loop's state for EOS at
the prefill pass, inside a group and at a group's last pass, over 1 and 3 rows;
a gated pass behind a closed gate changes nothing, in every kernel form."""
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


LOOPS = ["readback", "pinned", "pipelined"]


@pytest.mark.parametrize("loop", LOOPS)
@pytest.mark.parametrize("rng_mode", [S.RNG_XORSHIFT32, S.RNG_PHILOX], ids=["xorshift", "philox"])
def test_generate_matches_oracle_chain(rng_mode, loop):
    xs, params, hist = _inputs(21)
    max_new = 11  # prefill-final + groups of 4, 4, 2
    want, st = _oracle_chain(xs, params, hist, rng_mode, max_new)
    s = S.Sampler(V, 1)
    dev = [hip.DeviceBuffer.from_array(xs[k]) for k in range(NBUF)]
    pb = hip.PinnedBuffer(64) if loop != "readback" else None
    try:
        s.set_params(params, np.array([SEED], np.uint32))
        s.set_history(hist[None, :])
        table = G.LogitsTable([d.ptr for d in dev])
        toks, r = G.generate(s, table, max_new, rows=1, rng_mode=rng_mode, start_pos=START, pinned=pb,
                             pipelined=loop == "pipelined")
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


@pytest.mark.parametrize("loop", LOOPS)
def test_generate_stops_at_eos(loop):
    xs, params, hist = _inputs(22)
    want, _ = _oracle_chain(xs, params, hist, S.RNG_PHILOX, 9)
    eos = want[6]  # the sixth decode token (first occurrence decides)
    stop_at = want.index(eos) + 1
    s = S.Sampler(V, 1)
    dev = [hip.DeviceBuffer.from_array(xs[k]) for k in range(NBUF)]
    pb = hip.PinnedBuffer(64) if loop != "readback" else None
    try:
        s.set_params(params, np.array([SEED], np.uint32))
        s.set_history(hist[None, :])
        table = G.LogitsTable([d.ptr for d in dev])
        toks, r = G.generate(s, table, 50, rows=1, rng_mode=S.RNG_PHILOX, eos=eos, start_pos=START,
                             pinned=pb, pipelined=loop == "pipelined")
        assert toks == want[:stop_at]
        assert r["finish_reason"] == 0 and r["emitted"] == stop_at
    finally:
        s.close()
        for d in dev:
            d.free()
        if pb is not None:
            pb.free()


def _run_loop(xs, params, hist, rows, eos, max_new, loop, rng_mode=S.RNG_XORSHIFT32):
    s = S.Sampler(V, rows)
    dev = [hip.DeviceBuffer.from_array(np.ascontiguousarray(np.repeat(xs[k][None, :], rows, 0)))
           for k in range(NBUF)]
    pb = hip.PinnedBuffer(64 * rows) if loop != "readback" else None
    try:
        s.set_params(np.repeat(params, rows),
                     np.arange(SEED, SEED + rows, dtype=np.uint32))
        s.set_history(np.repeat(hist[None, :], rows, 0))
        table = G.LogitsTable([d.ptr for d in dev])
        toks, r = G.generate(s, table, max_new, rows=rows, rng_mode=rng_mode, eos=eos, start_pos=START,
                             pinned=pb, pipelined=loop == "pipelined")
        res, tk = s.read_results(rows)
        state = s.read_state(rows)
    finally:
        s.close()
        for d in dev:
            d.free()
        if pb is not None:
            pb.free()
    return toks, r, res, tk, state


@pytest.mark.parametrize("rows", [1, 3])
@pytest.mark.parametrize("where", ["prefill", "mid_group", "group_end", "none"])
def test_pipelined_matches_unpipelined_state(where, rows):
    """EOS at the prefill pass, inside a decode group, at a group's last pass,
    or never: the pipelined loop's tokens, result slots, token ids and final
    state equal the unpipelined loop's (the groups it queued past the EOS
    group did nothing)."""
    xs, params, hist = _inputs(23)
    ref, _ = _oracle_chain(xs, params, hist, S.RNG_XORSHIFT32, 14)
    idx = {"prefill": 0, "mid_group": 6, "group_end": 8, "none": None}[where]  # decode j -> index j + 1
    eos = ref[idx] if idx is not None else 0xFFFFFFFF
    print(f"pipelined eos={where} rows={rows}", flush=True)
    a = _run_loop(xs, params, hist, rows, eos, 14, "readback")
    b = _run_loop(xs, params, hist, rows, eos, 14, "pipelined")
    assert a[0] == b[0] == ref[:len(a[0])]
    assert a[1]["emitted"] == b[1]["emitted"] and a[1]["finish_reason"] == b[1]["finish_reason"]
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])
    for k in ("history", "position", "rng", "step"):
        assert np.array_equal(a[4][k], b[4][k]), k


@pytest.mark.parametrize("flags", [0, S.ENQ_FUSED, S.ENQ_SMALL, S.ENQ_SPLIT, S.ENQ_GENERAL, S.ENQ_RESIDENT],
                         ids=["auto", "fused", "small", "split", "general", "resident"])
def test_closed_gate_changes_nothing(flags):
    xs, params, hist = _inputs(24)
    rows = 2
    s = S.Sampler(V, rows)
    dev = hip.DeviceBuffer.from_array(np.ascontiguousarray(np.repeat(xs[0][None, :], rows, 0)))
    pb = hip.PinnedBuffer(64)
    try:
        s.set_params(np.repeat(params, rows), np.array([3, 4], np.uint32))
        s.set_history(np.repeat(hist[None, :], rows, 0))
        s.reset_gate()
        # pass 1 (sequence 1) draws row 0's token, which is the EOS id: it runs and closes the gate
        tok0 = O.o1_row(xs[0], params, O.RowState(hist.copy(), 0, 3, 0), want_kept=False)["token"]
        s.enqueue(dev.ptr, S.DTYPE_F32, V, rows, flags=flags | S.ENQ_GATED, gate_seq=1, eos=tok0,
                  pass_idx=1)
        res1, tk1 = s.read_results(rows)
        st1 = s.read_state(rows)
        assert int(tk1[0]) == tok0 and int(res1[0][1]) == tok0
        # a later pass of the same group (sequence 1) still runs
        s.enqueue(dev.ptr, S.DTYPE_F32, V, rows, flags=flags | S.ENQ_GATED, gate_seq=1, eos=tok0,
                  pass_idx=2)
        res2, tk2 = s.read_results(rows)
        st2 = s.read_state(rows)
        assert not np.array_equal(st2["position"], st1["position"])
        # the next group (sequence 2) does nothing: no slot, token, host token or state change
        host = pb.view(np.uint32, 16)
        host[:] = 0xABCDABCD
        s.enqueue(dev.ptr, S.DTYPE_F32, V, rows, flags=flags | S.ENQ_GATED, gate_seq=2, eos=tok0,
                  pass_idx=3, host_tokens=pb.dev_ptr)
        res3, tk3 = s.read_results(rows)
        st3 = s.read_state(rows)
        assert np.array_equal(res3, res2) and np.array_equal(tk3, tk2)
        assert np.all(host[:rows] == 0xABCDABCD)
        for k in ("history", "position", "rng", "step"):
            assert np.array_equal(st3[k], st2[k]), k
        # reopened, it runs again
        s.reset_gate()
        s.enqueue(dev.ptr, S.DTYPE_F32, V, rows, flags=flags | S.ENQ_GATED, gate_seq=2, eos=tok0, pass_idx=3)
        st4 = s.read_state(rows)
        assert not np.array_equal(st4["position"], st3["position"])
    finally:
        s.close()
        dev.free()
        pb.free()


@pytest.mark.parametrize("max_new", [1, 2, 5, 6])
def test_pipelined_short_runs(max_new):
    """Prefill only, one partial group, one full group, one full group plus a
    pass: the pipelined loop equals the unpipelined one (tokens, slots, state)."""
    xs, params, hist = _inputs(25)
    ref, _ = _oracle_chain(xs, params, hist, S.RNG_XORSHIFT32, max_new)
    a = _run_loop(xs, params, hist, 1, 0xFFFFFFFF, max_new, "readback")
    b = _run_loop(xs, params, hist, 1, 0xFFFFFFFF, max_new, "pipelined")
    assert a[0] == b[0] == ref
    assert a[1]["groups"] == b[1]["groups"] == (max_new - 1 + 3) // 4
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])
    for k in ("history", "position", "rng", "step"):
        assert np.array_equal(a[4][k], b[4][k]), k


@pytest.mark.parametrize("seed", range(10))
def test_random_decode_runs(seed):
    """Seeded random runs: 1..8 rows, 1..40 new tokens, either rng mode, EOS at
    a random point of the chain or never.  The three loops (slots read back per
    group, pinned tokens, pipelined) give the oracle chain's tokens, the same
    finish and the same result slots, token ids and final state."""
    rng = np.random.default_rng(300 + seed)
    rows = int(rng.integers(1, 9))
    max_new = int(rng.integers(1, 41))
    rng_mode = S.RNG_PHILOX if rng.random() < 0.5 else S.RNG_XORSHIFT32
    xs, params, hist = _inputs(100 + seed)
    ref, _ = _oracle_chain(xs, params, hist, rng_mode, max_new)
    idx = int(rng.integers(0, max_new)) if rng.random() < 0.6 else None
    eos = ref[idx] if idx is not None else 0xFFFFFFFF
    print(f"random decode {seed}: rows={rows} max_new={max_new} eos_index={idx}", flush=True)
    runs = [_run_loop(xs, params, hist, rows, eos, max_new, loop, rng_mode) for loop in LOOPS]
    a = runs[0]
    assert a[0] == ref[:len(a[0])]
    for b in runs[1:]:
        assert a[0] == b[0]
        assert a[1]["emitted"] == b[1]["emitted"] and a[1]["finish_reason"] == b[1]["finish_reason"]
        assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])
        for k in ("history", "position", "rng", "step"):
            assert np.array_equal(a[4][k], b[4][k]), k
