"""INTEGRATION.md's drop-in snippet, compiled as C11 and linked to the real
sampler library (tests/c/libsnippet_harness.so, built by build()), run on
the GPU as the reference runs a request (generatorSetSampling ->
resetGenerator's zero fill -> prefill-final pass -> decode groups;
src/compute.c:122-127, src/generate.c:1000-1016, :1118-1156, :1238-1252) and
checked against an O1 chain: every token, the final history ring,
position, rng and Philox step."""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from pumice_amd import hip
from pumice_amd import sampler as S

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "tests", "c", "libsnippet_harness.so")


def test_snippet_request_matches_oracle():
    if not os.path.exists(HARNESS):
        pytest.fail("tests/c/libsnippet_harness.so is missing: run build() (make -C tests/c)")
    S.lib()  # the sampler library the harness links against, loaded first
    L = ctypes.CDLL(HARNESS)
    P = ctypes.c_void_p
    L.snippet_chain.restype = ctypes.c_int
    L.snippet_chain.argtypes = [ctypes.c_uint32, P, ctypes.c_uint32, ctypes.c_uint32, P, ctypes.c_uint32, P, P, P]
    V, groups, seed, pos0 = 102400, 3, 12345, 7
    npass = 1 + 4 * groups
    rng = np.random.default_rng(77)
    x = (rng.standard_normal((npass, V)) * 3.0).astype(np.float32)
    x[:, 0] = np.float32(14.0)  # id 0 tops every row: the zero-filled window must penalize it
    p = S.make_params(1, temperature=0.8, repPenalty=1.3, penaltyLength=64, topK=40, topP=0.95,
                      minP=0.05, presencePenalty=0.5)
    dev = [hip.DeviceBuffer.from_array(x[k]) for k in range(npass)]
    try:
        ptrs = (ctypes.c_void_p * npass)(*[d.ptr for d in dev])
        tokens = np.zeros(npass, np.uint32)
        hist = np.zeros(S.MAX_PENALTY_LEN, np.uint32)
        state = np.zeros(3, np.uint32)
        st = L.snippet_chain(V, p.ctypes.data, seed, pos0, ptrs, groups, tokens.ctypes.data, hist.ctypes.data,
                             state.ctypes.data)
        assert st == 0, S.STATUS.get(st, st)
    finally:
        for d in dev:
            d.free()
    ost = O.RowState(np.zeros(S.MAX_PENALTY_LEN, np.uint32), pos0, seed, 0)
    for k in range(npass):
        want = O.o1_row(x[k], p[0], ost, do_increment=0 if k == 0 else 1, want_kept=False)["token"]
        assert int(tokens[k]) == want, f"pass {k}: snippet {tokens[k]} oracle {want}"
    assert int(state[0]) == ost.position and int(state[1]) == ost.rng and int(state[2]) == ost.step
    assert np.array_equal(hist, ost.history)
    assert int(tokens[0]) != 0, "id 0 sits in the zero-filled window: it must be penalized away"
