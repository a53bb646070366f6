"""GPU parity of the LM head (include/pumice_lmhead.h) against the oracle's
restatement in the same summation order: logits bit for bit (NaN compared as
NaN) over ragged vocabularies, K down to one 8-row block, 1..9 rows (row
groups of 1, 2 and 4 with a partial last group), K above the norm kernel's
single-pass size (4,104, 8,192), padded strides; the fused
greedy form against the oracle's argmax of those logits and against
pss_enqueue(PSS_MODE_GREEDY) on plh_logits' output (same token, result slot,
token_ids and position, nothing else touched); the reference validation case
(src/validation.c:4893-4941: position 41 -> 42); ties, NaN weights and zero
rows; two greedy calls in a row (the per-group tickets reset themselves);
plh_pack_head against the reference's load-time build restated in the oracle
(bf16 / fp16 rows, pruned by a map or not, format specials), then the logits of
a packed head; 12 seeded random shapes, strides and scales (logits and greedy)."""
import numpy as np
import pytest

import oracle as O
from pumice_amd import hip
from pumice_amd import lmhead as L
from pumice_amd import sampler as S

pytestmark = pytest.mark.gpu


def _same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _inputs(K, V, rows, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 2, (rows, K)).astype(np.float32)
    g = rng.normal(1, 0.3, K).astype(np.float32)
    w_kv = O.float_to_fp16((rng.normal(0, scale, (K, V))).astype(np.float32))
    return x, g, w_kv


def _oracle_logits(x, g, w_bt):
    out = []
    for r in range(x.shape[0]):
        _, a = O.lmhead_norm(x[r], g)
        out.append(O.lmhead_logits(a, w_bt))
    return np.stack(out)


class _Head:
    def __init__(self, x, g, w_bt, x_stride=None, max_rows=None):
        rows, K = x.shape
        self.K, self.V, self.rows = K, w_bt.shape[1], rows
        self.x_stride = x_stride or K
        xp = np.zeros((rows, self.x_stride), np.float32)
        xp[:, :K] = x
        self.dw = hip.DeviceBuffer.from_array(np.ascontiguousarray(w_bt))
        self.dg = hip.DeviceBuffer.from_array(g)
        self.dx = hip.DeviceBuffer.from_array(xp)
        self.h = L.LMHead(self.dw.ptr, self.dg.ptr, K, self.V, max_rows or rows)

    def logits(self, stride=None):
        stride = stride or self.V
        dl = hip.DeviceBuffer(self.rows * stride * 4)
        try:
            dl.fill_u32(0x7FC00001)
            self.h.logits(self.dx.ptr, self.x_stride, self.rows, dl.ptr, stride)
            hip.stream_sync(self.h.stream)
            out = dl.download(np.float32, (self.rows, stride))
        finally:
            dl.free()
        return out

    def close(self):
        self.h.close()
        for b in (self.dw, self.dg, self.dx):
            b.free()


@pytest.mark.parametrize("K,V,rows", [(8, 1, 1), (16, 63, 1), (24, 65, 2), (64, 1000, 3), (40, 129, 4),
                                      (512, 4096, 5), (256, 3000, 9), (4096, 32768, 2), (4104, 777, 2),
                                      (8192, 3000, 1)])
def test_logits_bit_exact(K, V, rows):
    x, g, w_kv = _inputs(K, V, rows, seed=K * 7 + V + rows)
    w_bt = O.transpose_block16(w_kv)
    print(f"lmhead logits K={K} V={V} rows={rows}", flush=True)
    hd = _Head(x, g, w_bt)
    try:
        got = hd.logits()
    finally:
        hd.close()
    want = _oracle_logits(x, g, w_bt)
    for r in range(rows):
        assert _same(got[r], want[r]), (r, np.flatnonzero(got[r] != want[r])[:8])


def test_logits_padded_strides():
    K, V, rows = 128, 777, 3
    x, g, w_kv = _inputs(K, V, rows, seed=11)
    w_bt = O.transpose_block16(w_kv)
    hd = _Head(x, g, w_bt, x_stride=K + 13)
    try:
        got = hd.logits(stride=V + 5)
    finally:
        hd.close()
    want = _oracle_logits(x, g, w_bt)
    assert _same(got[:, :V], want)
    assert np.all(got[:, V:].view(np.uint32) == 0x7FC00001)  # padding untouched


def _greedy_run(x, g, w_bt, pass_idx=0, do_increment=1, calls=1):
    rows, K = x.shape
    V = w_bt.shape[1]
    hd = _Head(x, g, w_bt)
    s = S.Sampler(V, rows, stream=hd.h.stream)
    try:
        s.set_position(np.full(rows, 41, np.uint32))
        before = s.read_state(rows)
        for _ in range(calls):
            hd.h.greedy(s, hd.dx.ptr, K, rows, do_increment=do_increment, pass_idx=pass_idx)
        res, tok = s.read_results(rows)
        after = s.read_state(rows)
    finally:
        s.close()
        hd.close()
    return res, tok, before, after


@pytest.mark.parametrize("K,V,rows", [(8, 7, 1), (64, 1000, 1), (128, 5000, 2), (96, 2049, 3), (512, 20000, 6)])
def test_greedy_matches_oracle(K, V, rows):
    x, g, w_kv = _inputs(K, V, rows, seed=K + V * 3 + rows)
    w_bt = O.transpose_block16(w_kv)
    print(f"lmhead greedy K={K} V={V} rows={rows}", flush=True)
    res, tok, before, after = _greedy_run(x, g, w_bt, pass_idx=2)
    want = _oracle_logits(x, g, w_bt)
    for r in range(rows):
        t = O.greedy(want[r])
        assert int(tok[r]) == t and int(res[r][2]) == t
        assert t == O.greedy_two_stage(want[r])  # the reference's two-stage tree on the same logits
    assert np.array_equal(after["position"], before["position"] + 1)
    assert np.array_equal(after["history"], before["history"])
    assert np.array_equal(after["rng"], before["rng"]) and np.array_equal(after["step"], before["step"])


def test_greedy_equals_logits_then_sampler_greedy():
    K, V, rows = 256, 9000, 3
    x, g, w_kv = _inputs(K, V, rows, seed=77)
    w_bt = O.transpose_block16(w_kv)
    hd = _Head(x, g, w_bt)
    s1 = S.Sampler(V, rows, stream=hd.h.stream)
    s2 = S.Sampler(V, rows, stream=hd.h.stream)
    dl = hip.DeviceBuffer(rows * V * 4)
    try:
        hd.h.greedy(s1, hd.dx.ptr, K, rows, do_increment=0, pass_idx=1)
        hd.h.logits(hd.dx.ptr, K, rows, dl.ptr, V)
        s2.enqueue(dl.ptr, S.DTYPE_F32, V, rows, S.MODE_GREEDY, 0, 1, S.RNG_XORSHIFT32)
        r1, t1 = s1.read_results(rows)
        r2, t2 = s2.read_results(rows)
        st1, st2 = s1.read_state(rows), s2.read_state(rows)
    finally:
        s1.close()
        s2.close()
        dl.free()
        hd.close()
    assert np.array_equal(t1, t2) and np.array_equal(r1[:, 1], r2[:, 1])
    for k in ("history", "position", "rng", "step"):
        assert np.array_equal(st1[k], st2[k])


def test_reference_validation_case():
    """src/validation.c:6113-6116, :6174-6175, :4893-4941: K = 4096, V = 102,400,
    one row; the token equals the oracle's and position goes 41 -> 42."""
    K, V = 4096, 102400
    x = O.get_data(4321, 1, K)
    g = O.get_data(58923, 1, K)[0]
    w_bt = O.transpose_block16(O.get_data_fp16(15001, K, V))
    print("lmhead reference validation case", flush=True)
    want = _oracle_logits(x, g, w_bt)[0]
    hd = _Head(x, g, w_bt)
    try:
        got = hd.logits()[0]
    finally:
        hd.close()
    assert _same(got, want)
    res, tok, before, after = _greedy_run(x, g, w_bt)
    assert int(tok[0]) == O.greedy(want) == int(res[0][0])
    assert int(after["position"][0]) == 42


def test_ties_nan_and_zero_rows():
    K, V = 64, 300
    rng = np.random.default_rng(9)
    g = np.ones(K, np.float32)
    x = rng.normal(0, 1, (3, K)).astype(np.float32)
    x[2] = 0.0                                        # zero row: all logits 0 -> token 0
    w_kv = O.float_to_fp16(rng.normal(0, 1, (K, V)).astype(np.float32))
    _, a0 = O.lmhead_norm(x[0], g)
    best = int(np.argmax(O.lmhead_logits(a0, O.transpose_block16(w_kv))))
    tie = 299 if best != 299 else 0
    nan_col = 17 if best != 17 else 18
    w_kv[:, tie] = w_kv[:, best]                      # a tie of row 0's maximum
    w_kv[:, nan_col] = 0x7E00                         # a NaN column never wins
    w_bt = O.transpose_block16(w_kv)
    want = _oracle_logits(x, g, w_bt)
    assert np.isnan(want[0, nan_col]) and want[0, tie] == want[0, best]
    res, tok, _, _ = _greedy_run(x, g, w_bt)
    assert int(tok[0]) == min(best, tie) == O.greedy(want[0])
    assert int(tok[1]) == O.greedy(want[1])
    assert int(tok[2]) == 0 == O.greedy(want[2])


def test_greedy_twice_in_a_row():
    K, V, rows = 64, 4100, 5
    x, g, w_kv = _inputs(K, V, rows, seed=5)
    w_bt = O.transpose_block16(w_kv)
    res, tok, before, after = _greedy_run(x, g, w_bt, calls=2)
    want = _oracle_logits(x, g, w_bt)
    assert [int(t) for t in tok] == [O.greedy(want[r]) for r in range(rows)]
    assert np.array_equal(after["position"], before["position"] + 2)


def test_argument_errors():
    K, V = 16, 10
    x, g, w_kv = _inputs(K, V, 1, seed=1)
    hd = _Head(x, g, O.transpose_block16(w_kv))
    s_other = S.Sampler(V, 1)           # its own stream
    s_wrong_v = S.Sampler(V + 1, 1, stream=hd.h.stream)
    try:
        with pytest.raises(S.PssError):
            hd.h.logits(hd.dx.ptr, K - 1, 1, hd.dx.ptr, V)          # x_stride < K
        with pytest.raises(S.PssError):
            hd.h.logits(hd.dx.ptr, K, 2, hd.dx.ptr, V)              # rows > max_rows
        with pytest.raises(S.PssError):
            hd.h.greedy(s_other, hd.dx.ptr, K, 1)                   # different stream
        with pytest.raises(S.PssError):
            hd.h.greedy(s_wrong_v, hd.dx.ptr, K, 1)                 # different vocabulary
        with pytest.raises(S.PssError):
            L.LMHead(hd.dw.ptr, hd.dg.ptr, 12, V, 1)                # K % 8 != 0
    finally:
        s_other.close()
        s_wrong_v.close()
        hd.close()


def _src_rows(rng, rows, K, dtype):
    bits = rng.integers(0, 65536, (rows, K), dtype=np.uint32).astype(np.uint16)
    # specials of the source format: NaN, +-inf, zeros, subnormals, values past fp16's range
    if dtype == L.SRC_FP16:
        sp = [0x7E00, 0x7C00, 0xFC00, 0x0000, 0x8000, 0x0001, 0x03FF, 0x7BFF]
    else:
        sp = [0x7FC0, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x477F, 0x4780, 0x3380]
    flat = bits.reshape(-1)
    n = min(len(sp), flat.size)
    flat[:n] = sp[:n]
    return bits


@pytest.mark.parametrize("dtype", [0, 1], ids=["bf16", "fp16"])
@pytest.mark.parametrize("mapped", [True, False], ids=["pruned", "unpruned"])
@pytest.mark.parametrize("K,V", [(24, 65), (264, 1000), (8, 1)])
def test_pack_head_bit_exact(dtype, mapped, K, V):
    rng = np.random.default_rng(K + V + 2 * dtype + mapped)
    src_rows = V + 300 if mapped else V
    src = _src_rows(rng, src_rows, K, dtype)
    mapping = rng.permutation(src_rows)[:V].astype(np.int32) if mapped else None
    if mapped:
        mapping[:2] = [0, 1][:V]  # the rows holding the specials
    want = O.pack_head(src, dtype, mapping)
    print(f"pack_head dtype={dtype} mapped={mapped} K={K} V={V}", flush=True)
    ds = hip.DeviceBuffer.from_array(src)
    dw = hip.DeviceBuffer(K * V * 2)
    try:
        L.pack_head(ds.ptr, dtype, src_rows, K, mapping, V, dw.ptr)
        got = dw.download(np.uint16, (K // 8, V, 8))
    finally:
        ds.free()
        dw.free()
    assert np.array_equal(got, want), np.argwhere(got != want)[:5]


def test_pack_then_logits():
    """bf16 lm_head rows of a 2,000-row vocabulary, pruned to 777 ids, packed on
    the GPU, then plh_logits: the logits equal the oracle's on the oracle's
    packed head."""
    rng = np.random.default_rng(21)
    K, V, src_rows = 256, 777, 2000
    src = O.float_to_bf16(rng.normal(0, 0.05, (src_rows, K)).astype(np.float32))
    mapping = rng.permutation(src_rows)[:V].astype(np.int32)
    w_bt = O.pack_head(src, 0, mapping)
    x = rng.normal(0, 2, (2, K)).astype(np.float32)
    g = rng.normal(1, 0.2, K).astype(np.float32)
    ds = hip.DeviceBuffer.from_array(src)
    dw = hip.DeviceBuffer(K * V * 2)
    dg, dx = hip.DeviceBuffer.from_array(g), hip.DeviceBuffer.from_array(x)
    dl = hip.DeviceBuffer(2 * V * 4)
    try:
        L.pack_head(ds.ptr, 0, src_rows, K, mapping, V, dw.ptr)
        h = L.LMHead(dw.ptr, dg.ptr, K, V, 2)
        try:
            h.logits(dx.ptr, K, 2, dl.ptr, V)
            hip.stream_sync(h.stream)
        finally:
            h.close()
        got = dl.download(np.float32, (2, V))
    finally:
        for b in (ds, dw, dg, dx, dl):
            b.free()
    assert _same(got, _oracle_logits(x, g, w_bt))


def test_pack_head_errors():
    src = np.zeros((10, 16), np.uint16)
    ds = hip.DeviceBuffer.from_array(src)
    dw = hip.DeviceBuffer(16 * 12 * 2)
    try:
        with pytest.raises(S.PssError):   # map entry past the source rows (src/prune.c:159-161)
            L.pack_head(ds.ptr, 0, 10, 16, np.array([0, 10], np.int32), 2, dw.ptr)
        with pytest.raises(S.PssError):   # negative entry
            L.pack_head(ds.ptr, 0, 10, 16, np.array([-1], np.int32), 1, dw.ptr)
        with pytest.raises(S.PssError):   # unpruned with fewer source rows than V
            L.pack_head(ds.ptr, 0, 10, 16, None, 12, dw.ptr)
        with pytest.raises(S.PssError):   # K % 8 != 0
            L.pack_head(ds.ptr, 0, 10, 12, None, 10, dw.ptr)
        with pytest.raises(S.PssError):   # source not 16-byte aligned
            L.pack_head(ds.ptr + 2, 0, 9, 16, None, 9, dw.ptr)
    finally:
        ds.free()
        dw.free()


def _random_head_case(seed):
    rng = np.random.default_rng(500 + seed)
    K = 8 * int(rng.integers(1, 513))
    V = int(rng.integers(1, 40001))
    rows = int(rng.integers(1, 9))
    x = (rng.normal(0, rng.uniform(0.01, 10.0), (rows, K))).astype(np.float32)
    if rows > 1 and rng.random() < 0.3:
        x[int(rng.integers(0, rows))] = 0.0             # a zero row: every logit 0, token 0
    g = rng.normal(1, rng.uniform(0.0, 1.0), K).astype(np.float32)
    if rng.random() < 0.3:                               # few distinct weights: tied logits
        w = rng.integers(-3, 4, (K, V)).astype(np.float32) * np.float32(0.125)
    else:
        w = rng.normal(0, rng.uniform(0.001, 2.0), (K, V)).astype(np.float32)
    return x, g, O.float_to_fp16(w)


@pytest.mark.parametrize("seed", range(12))
def test_random_heads(seed):
    """Seeded random shapes (K from 8 to 4,096, V from 1 to 40,000, 1..8 rows),
    padded strides, activation and weight scales over several decades, tied
    and zero rows: logits bit-exact, then the fused greedy form's tokens."""
    x, g, w_kv = _random_head_case(seed)
    rows, K = x.shape
    V = w_kv.shape[1]
    rng = np.random.default_rng(seed)
    x_stride = K + 4 * int(rng.integers(0, 3))
    l_stride = V + int(rng.integers(0, 5))
    print(f"lmhead random {seed}: K={K} V={V} rows={rows} strides {x_stride}/{l_stride}", flush=True)
    w_bt = O.transpose_block16(w_kv)
    want = _oracle_logits(x, g, w_bt)
    hd = _Head(x, g, w_bt, x_stride=x_stride)
    try:
        got = hd.logits(stride=l_stride)
    finally:
        hd.close()
    assert _same(got[:, :V], want)
    res, tok, before, after = _greedy_run(x, g, w_bt, pass_idx=1)
    assert [int(t) for t in tok] == [O.greedy(want[r]) for r in range(rows)]
    assert [int(r[1]) for r in res] == [int(t) for t in tok]
    assert np.array_equal(after["position"], before["position"] + 1)
