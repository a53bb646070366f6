"""GPU parity of the request sequence around the sampler step and of a long
decode chain, through the C ABI against O1:

- resetGenerator's window reset (src/generate.c:1238-1252): pss_reset_history
  on a row range that starts above row 0, with the reference's zero fill
  (src/buffer.c:233-239, so id 0 is penalized until the window has been
  overwritten by sampled tokens) and with the empty-slot sentinel; then the
  prefill-final pass (doIncrement = 0, src/generate.c:1000-1016) and decode
  passes.  Rows outside the range keep their windows.  Every kernel form.
- the full 1,000-step batch-1 chain of the latency configuration (V =
  102,400 fp32 ~ N(0, 3^2), a fresh row per step, rep 1.1 / presence 0.5
  over a 64-id window, T 0.8, top-k 40, top-p 0.95, min-p 0.05, Philox key 0
  with the step as counter): every token, and the final window ring,
  position and Philox step, as the reference's validator checks chained
  draws and their side effects (src/validation.c:5141-5178)."""
import numpy as np
import pytest

import oracle as O
from harness import GpuRun, OracleRun, compare_state, compare_step
from pumice_amd import hip
from pumice_amd import sampler as S
from pumice_amd import workloads as WL

pytestmark = pytest.mark.gpu

PATHS = [0, S.ENQ_FUSED, S.ENQ_SMALL, S.ENQ_SPLIT, S.ENQ_GENERAL, S.ENQ_RESIDENT]
PATH_IDS = ["auto", "fused", "small", "split", "general", "resident"]


def _reset_inputs(V, rows, W, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, (4, rows, V)).astype(np.float32)
    # id 0 carries the row maximum, so whether it is penalized decides the
    # row maximum, the kept set and usually the token
    x[:, :, 0] = np.float32(15.0)
    params = O.make_params(temperature=0.8, repPenalty=1.3, presencePenalty=0.8, penaltyLength=W,
                           topK=40, topP=0.95, minP=0.0, rows=rows)
    hist = np.full((rows, O.MAX_PEN), O.SENTINEL, np.uint32)
    hist[:, :W] = rng.integers(1, V, (rows, W), dtype=np.uint32)
    seeds = rng.integers(1, 2**32, rows, dtype=np.uint32)
    return x, params, hist, seeds


@pytest.mark.parametrize("fill", [0, O.SENTINEL], ids=["zero_fill", "sentinel_fill"])
@pytest.mark.parametrize("flags", PATHS, ids=PATH_IDS)
def test_reset_prefill_decode(fill, flags):
    V, rows, W, row0, nreset, P = 102400, 6, 32, 2, 3, 5
    x, params, hist, seeds = _reset_inputs(V, rows, W, seed=11)
    g = GpuRun(x[0], params, seeds, hist, np.full(rows, P, np.uint32))
    ohist = hist.copy()
    ohist[row0:row0 + nreset] = fill
    o = OracleRun(rows, params, seeds, ohist, np.full(rows, P, np.uint32))
    try:
        g.s.reset_history(fill, row0=row0, rows=nreset)
        st = g.state()
        assert np.all(st["history"][row0:row0 + nreset] == fill)
        assert np.array_equal(st["history"][:row0], hist[:row0])
        assert np.array_equal(st["history"][row0 + nreset:], hist[row0 + nreset:])
        infos = []
        for k in range(4):  # prefill-final pass, then three decode passes
            inc = 0 if k == 0 else 1
            g.load(x[k])
            go = g.step(do_increment=inc, pass_idx=k % 4, flags=flags)
            oo = o.step(x[k], do_increment=inc)
            compare_step(go, oo, pass_idx=k % 4, where=f"fill {fill:#x} pass {k}")
            infos.append(go["info"])
        compare_state(g.state(), o, where=f"fill {fill:#x}")
        # id 0 holds the row maximum of the raw logits; the transform is
        # l * (1 / T) in binary32.  Zero fill: id 0 is in every reset window
        # and penalized, so the maximum is another id's.  Sentinel fill: id 0
        # is in no window (the loaded windows hold ids >= 1).
        k0 = O.key(np.float32(15.0) * (np.float32(1.0) / np.float32(0.8)))
        for r in range(row0, row0 + nreset):
            tk = int(infos[0][r]["tmax_key"])
            if fill == 0:
                assert tk != k0, f"row {r}: id 0 not penalized after the zero fill"
            else:
                assert tk == k0, f"row {r}: id 0 penalized after the sentinel fill"
    finally:
        g.close()


def _c2_rows(seed, steps, V):
    """A fresh N(0, 3^2) logit row per step (generated one at a time)."""
    rng = np.random.default_rng(seed)
    for _ in range(steps):
        yield WL.normal_rows(rng, 1, V, 3.0)[0]


def test_c2_full_chain_1000_steps():
    steps, V = 1000, WL.V_PRUNED
    w, _ = WL.c2(seed=2, rows=1, steps=1)
    seeds = np.zeros(1, np.uint32)  # Philox key 0, counter = (step, row 0)
    s = S.Sampler(V, 1)
    dev = hip.DeviceBuffer(V * 4)
    st = O.RowState(w.history[0], 0, 0, 0)
    try:
        s.set_params(w.params, seeds)
        s.set_history(w.history)
        got, want = [], []
        for k, x in enumerate(_c2_rows(1000 + 2, steps, V)):
            dev.upload(x)
            s.enqueue(dev.ptr, S.DTYPE_F32, V, 1, rng_mode=S.RNG_PHILOX)
            _, tok = s.read_results(1)
            got.append(int(tok[0]))
            want.append(O.o1_row(x, w.params[0], st, rng_mode=1, want_kept=False)["token"])
            assert got[-1] == want[-1], f"step {k}: gpu {got[-1]} oracle {want[-1]}"
        fin = s.read_state(1)
        assert int(fin["position"][0]) == st.position == steps
        assert int(fin["step"][0]) == st.step == steps
        assert int(fin["rng"][0]) == st.rng
        assert np.array_equal(fin["history"][0], st.history)
        # the ring holds the last 64 sampled tokens in slot order
        for k in range(steps - 64, steps):
            assert int(fin["history"][0, k % 64]) == got[k]
        assert len(set(got)) > 500, "draws should vary across fresh rows"
    finally:
        s.close()
        dev.free()
