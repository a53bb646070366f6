"""pss_enqueue_noalloc (the entry point that allocates nothing: its workspace
is a per-GPU array inside the library) against pss_enqueue_ex on the same
inputs, bit for bit: tokens, result slots, row diagnostics and the per-row
state, on two calls in a row, the second with fewer rows."""
import numpy as np
import pytest

from pumice_amd import hip
from pumice_amd import sampler as S

pytestmark = pytest.mark.gpu

V = 102400


def _params(rows, rng):
    p = S.make_params(rows, temperature=0.8, repPenalty=1.1, presencePenalty=0.5, penaltyLength=64,
                      topK=40, topP=0.95, minP=0.05)
    p[1]["temperature"] = 0.0                      # greedy row
    p[2]["topK"] = 300                              # above the streaming forms' top-k cover
    p[3]["penaltyLength"] = 700                     # wide window
    p[4]["topP"] = 0.5
    p[5]["minP"] = 0.0
    p[6]["topK"] = 1
    return p


def _state(s, rows):
    st = s.read_state(rows)
    res, tok = s.read_results(rows)
    return st, res, tok


def test_noalloc_matches_enqueue_ex_two_calls():
    rows = S.NOALLOC_MAX_ROWS
    rng = np.random.default_rng(5)
    params = _params(rows, rng)
    seeds = rng.integers(1, 2**32, rows, dtype=np.uint32)
    hist = np.full((rows, S.MAX_PENALTY_LEN), S.SENTINEL, np.uint32)
    hist[:, :700] = rng.integers(0, V, (rows, 700), dtype=np.uint32)
    s = S.Sampler(V, rows)
    bufs = []
    try:
        s.set_params(params, seeds)
        s.set_history(hist)
        st0, res0, tok0 = _state(s, rows)
        # the caller's own buffers for the allocation-free call, same contents
        dev = {
            "result": hip.DeviceBuffer.from_array(res0),
            "token_ids": hip.DeviceBuffer.from_array(tok0),
            "position": hip.DeviceBuffer.from_array(st0["position"]),
            "rng": hip.DeviceBuffer.from_array(st0["rng"]),
            "step": hip.DeviceBuffer.from_array(st0["step"]),
            "history": hip.DeviceBuffer.from_array(st0["history"]),
        }
        bufs += list(dev.values())
        pdev = hip.DeviceBuffer.from_array(np.ascontiguousarray(params))
        info_a = hip.DeviceBuffer(rows * S.ROW_INFO.itemsize)
        info_b = hip.DeviceBuffer(rows * S.ROW_INFO.itemsize)
        bufs += [pdev, info_a, info_b]
        ptrs = {k: b.ptr for k, b in dev.items()}
        for call, (n, pass_idx, mode) in enumerate([(rows, 0, S.RNG_PHILOX), (5, 1, S.RNG_XORSHIFT32)]):
            x = (rng.standard_normal((rows, V)) * 3.0).astype(np.float32)
            xd = hip.DeviceBuffer.from_array(x)
            bufs.append(xd)
            s.enqueue(xd.ptr, S.DTYPE_F32, V, n, pass_idx=pass_idx, rng_mode=mode, row_info=info_a.ptr)
            hip.synchronize()
            S.enqueue_noalloc(pdev.ptr, ptrs, V, xd.ptr, S.DTYPE_F32, V, n, pass_idx=pass_idx, rng_mode=mode,
                              max_topk=300, max_window=700, row_info=info_b.ptr)
            hip.synchronize()
            st, res, tok = _state(s, rows)
            where = f"call {call} ({n} rows)"
            assert np.array_equal(dev["token_ids"].download(np.uint32, rows), tok), where
            assert np.array_equal(dev["result"].download(np.uint32, (rows, S.RESULT_SLOTS)), res), where
            for k in ("position", "rng", "step"):
                assert np.array_equal(dev[k].download(np.uint32, rows), st[k]), f"{where}: {k}"
            assert np.array_equal(dev["history"].download(np.uint32, (rows, S.MAX_PENALTY_LEN)), st["history"]), where
            ia = info_a.download(S.ROW_INFO, rows)[:n]
            ib = info_b.download(S.ROW_INFO, rows)[:n]
            assert ia.tobytes() == ib.tobytes(), f"{where}: row info"
    finally:
        s.close()
        for b in bufs:
            b.free()
