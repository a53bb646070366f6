"""Pins of the LM-head restatement in oracle/ (no GPU): the fp16 helpers and
transpose_block16 against the reference's own src/data.c (golden fixture, and
the compiled oracle/_ref/ where present), fp16 -> fp32 against numpy over all
65,536 patterns, the RMSNorm against the binary64 formula and closed forms, the
GEMV against a numpy binary64 product of the untransposed matrix (a
transposed or dropped term fails the bound), one-hot columns, and the
reference validation case (src/validation.c:6113-6116, :6174-6175, :4893-4941)."""
import json
import math
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = json.load(open(os.path.join(HERE, "golden", "fp16_data.json")))
U = 2.0 ** -24


def test_float_to_fp16_matches_reference_fixture():
    f = np.array(FIX["float_to_fp16"]["in_bits"], np.uint32).view(np.float32)
    assert O.float_to_fp16(f).tolist() == FIX["float_to_fp16"]["out_bits"]


def test_float_to_fp16_truncates():
    """Mathematical pin: exact for every fp16 value, else the fp16 neighbour
    toward zero (|h| <= |f| < next fp16 up), saturating to inf at 2^16."""
    h = np.arange(0, 0x7C00, dtype=np.uint16)             # every finite non-negative half
    f = h.view(np.float16).astype(np.float32)
    assert np.array_equal(O.float_to_fp16(f), h)
    assert np.array_equal(O.float_to_fp16(-f), h | 0x8000)
    rng = np.random.default_rng(1)
    x = np.abs(rng.normal(0, 1000, 20000)).astype(np.float32)
    x = x[(x < 65504) & (x > 2.0 ** -24)]
    got = O.float_to_fp16(x).view(np.float16).astype(np.float64)
    nxt = (O.float_to_fp16(x) + 1).view(np.float16).astype(np.float64)
    assert np.all(got <= x) and np.all(x < nxt)
    assert O.float_to_fp16(np.array([65536.0, 1e9], np.float32)).tolist() == [0x7C00, 0x7C00]


def test_fp16_to_float_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.fp16_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_get_data_fp16_matches_reference_fixture():
    g = FIX["get_data_fp16"]
    K, V = g["M"], g["N"]
    for (i, j), bits in zip(g["pos"], g["bits"]):
        assert O.float_to_fp16(np.array([O.lib().oracle_get_pseudo_random(i, j, g["seed"])], np.float32))[0] == bits
    small = O.get_data_fp16(g["seed"], 2, V)
    for (i, j), bits in zip(g["pos"], g["bits"]):
        if i < 2:
            assert int(small[i, j]) == bits


def test_transpose_block16_matches_reference_fixture_and_reshape():
    t = FIX["transpose_block16"]
    K, V = t["K"], t["V"]
    w = np.array(t["in"], np.uint16).reshape(K, V)
    got = O.transpose_block16(w)
    assert got.reshape(-1).tolist() == t["out"]
    # independent statement of the layout: block (kb, n) = column n of rows 8kb..8kb+7
    assert np.array_equal(got, w.reshape(K // 8, 8, V).transpose(0, 2, 1))


def test_transpose_block16_against_compiled_reference():
    ref = O.ref_data_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    import ctypes
    ref.transpose_block16.restype = None
    ref.transpose_block16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    rng = np.random.default_rng(2)
    for K, V in [(8, 1), (32, 77), (64, 300)]:
        w = rng.integers(0, 65536, (K, V), dtype=np.uint16)
        out = np.zeros(K * V, np.uint16)
        ref.transpose_block16(w.ctypes.data, out.ctypes.data, K, V, 16)
        assert np.array_equal(O.transpose_block16(w).reshape(-1), out)


def test_lmhead_norm_pins():
    rng = np.random.default_rng(3)
    for K in [8, 24, 512, 4096]:
        x = rng.normal(0, 2, K).astype(np.float32)
        g = rng.normal(1, 0.2, K).astype(np.float32)
        inv, a = O.lmhead_norm(x, g)
        # the binary64 sum rounded once equals binary32 of the exact sum (fsum)
        ss = np.float32(math.fsum(float(v) * float(v) for v in x))
        want = np.float32(1.0) / np.sqrt(ss / np.float32(K) + np.float32(1e-6))
        assert np.float32(inv) == want
        exact = 1.0 / math.sqrt(math.fsum(float(v) ** 2 for v in x) / K + 1e-6)
        assert abs(inv - exact) <= 4 * U * exact
        assert np.array_equal(a, (x * g) * np.float32(inv))
    # closed forms: constant rows, zero rows
    inv, a = O.lmhead_norm(np.full(64, 3.0, np.float32), np.ones(64, np.float32))
    assert abs(inv - 1.0 / math.sqrt(9.0 + 1e-6)) <= 2 * U
    inv, a = O.lmhead_norm(np.zeros(16, np.float32), np.ones(16, np.float32))
    assert np.float32(inv) == np.float32(1.0) / np.sqrt(np.float32(1e-6)) and not a.any()


@pytest.mark.parametrize("K,V", [(8, 5), (64, 130), (512, 1000)])
def test_lmhead_logits_against_float64_product(K, V):
    rng = np.random.default_rng(K + V)
    a = rng.normal(0, 1, K).astype(np.float32)
    w_kv = O.float_to_fp16(rng.normal(0, 1, (K, V)).astype(np.float32))
    w_bt = O.transpose_block16(w_kv)
    wf = O.fp16_to_float(w_kv).astype(np.float64)
    exact = a.astype(np.float64) @ wf
    absdot = np.abs(a.astype(np.float64)) @ np.abs(wf)
    got = O.lmhead_logits(a, w_bt).astype(np.float64)
    # an fmaf chain of K/4 terms plus 3 additions: at most (K/4 + 3) u sum|a w|
    assert np.all(np.abs(got - exact) <= (K / 4 + 4) * U * absdot)
    g64, ad64 = O.lmhead_logits64(a, w_bt)
    assert np.allclose(g64, exact, rtol=0, atol=1e-12 * (1 + absdot.max()))
    assert np.allclose(ad64, absdot, rtol=1e-12)
    # a dropped block term or a transposed operand is far outside the bound
    bad = exact - a[5].astype(np.float64) * wf[5]
    assert np.any(np.abs(got - bad) > (K / 4 + 4) * U * absdot)


def test_lmhead_logits_one_hot_columns():
    """Column n = e_{k(n)}: every logit is exactly a[k(n)], in any order."""
    K, V = 64, 200
    rng = np.random.default_rng(7)
    a = rng.normal(0, 1, K).astype(np.float32)
    ks = rng.integers(0, K, V)
    w_kv = np.zeros((K, V), np.uint16)
    w_kv[ks, np.arange(V)] = 0x3C00  # 1.0
    got = O.lmhead_logits(a, O.transpose_block16(w_kv))
    assert np.array_equal(got, a[ks])
    for slices in (1, 2, 3, 4):
        assert np.array_equal(O.lmhead_logits(a, O.transpose_block16(w_kv), slices=slices), a[ks])


def test_reference_validation_case():
    """src/validation.c: K = 4096, input = getData(4321, 1, K), gamma =
    getData(58923, 1, K), head = getDataFP16(15001, K, 102400); the check
    compares the shader's token with lmhead_argmax_ref_fp16 (fp32 sequential
    mul + add, :3898-3910) over rms_norm_apply (:157-163).  The oracle's argmax
    in the GPU's order, the binary64 argmax and that fp32 sequential order
    (restated here in numpy) agree, with the top-2 gap far above the
    differences between the orders."""
    K, V = 4096, 102400
    x = O.get_data(4321, 1, K)[0]
    g = O.get_data(58923, 1, K)[0]
    w_kv = O.get_data_fp16(15001, K, V)
    w_bt = O.transpose_block16(w_kv)
    _, a = O.lmhead_norm(x, g)
    lo = O.lmhead_logits(a, w_bt)
    l64, absdot = O.lmhead_logits64(a, w_bt)
    tok = O.greedy(lo)
    assert tok == int(np.argmax(l64))
    # rms_norm_apply + lmhead_argmax_ref_fp16: binary32 throughout, sequential
    ss = np.float32(0.0)
    for v in x:
        ss = np.float32(ss + v * v)
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(K) + np.float32(1e-6))
    xn = (x * g) * inv
    acc = np.zeros(V, np.float32)
    for k in range(K):
        acc = acc + xn[k] * O.fp16_to_float(w_kv[k])
    assert int(np.argmax(acc)) == tok
    srt = np.sort(l64)
    err = max(np.abs(lo - l64).max(), np.abs(acc - l64).max())
    assert srt[-1] - srt[-2] > 20 * err


def test_float_to_bf16_matches_reference_fixture():
    f = np.array(FIX["float_to_bf16"]["in_bits"], np.uint32).view(np.float32)
    assert O.float_to_bf16(f).tolist() == FIX["float_to_bf16"]["out_bits"]


def test_float_to_bf16_rounds_to_nearest_even():
    """Mathematical pin: the nearer of the two bf16 neighbours, the one with
    an even last bit on a tie (finite values below the bf16 overflow)."""
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.normal(0, 100, 20000), rng.uniform(-1e-30, 1e-30, 2000)]).astype(np.float32)
    ties = (rng.integers(0, 1 << 16, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    b = x.view(np.uint32)
    lo = (b & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((b & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    dlo, dhi = np.abs(xd - lo), np.abs(hi - xd)
    lo_even = ((b >> 16) & 1) == 0
    pick_lo = (dlo < dhi) | ((dlo == dhi) & lo_even)
    want = np.where(pick_lo, b >> 16, (b >> 16) + 1).astype(np.uint16)
    assert np.array_equal(O.float_to_bf16(x), want)


def _ref_compose_pack(ref, src, dtype, mapping):
    """The reference's own data.c functions composed as prune.c + weights.c do."""
    import ctypes
    ref.float_to_fp16.restype = ctypes.c_uint16
    ref.float_to_fp16.argtypes = [ctypes.c_float]
    ref.fp16_to_float.restype = ctypes.c_float
    ref.fp16_to_float.argtypes = [ctypes.c_uint16]
    ref.float_to_bf16.restype = ctypes.c_uint16
    ref.float_to_bf16.argtypes = [ctypes.c_float]
    ref.bf16_to_float.restype = ctypes.c_float
    ref.bf16_to_float.argtypes = [ctypes.c_uint16]
    ref.transpose_block16.restype = None
    ref.transpose_block16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    rows = mapping if mapping is not None else np.arange(src.shape[0])
    V, K = len(rows), src.shape[1]
    eng = np.zeros((K, V), np.uint16)
    for v, r in enumerate(rows):
        for k in range(K):
            raw = int(src[r, k])
            if dtype == 0:
                x = ref.bf16_to_float(raw)
            elif mapping is not None:
                x = ref.bf16_to_float(ref.float_to_bf16(ref.fp16_to_float(raw)))
            else:
                x = ref.fp16_to_float(raw)
            eng[k, v] = ref.float_to_fp16(x)
    out = np.zeros(K * V, np.uint16)
    ref.transpose_block16(eng.ctypes.data, out.ctypes.data, K, V, 16)
    return out


@pytest.mark.parametrize("dtype,mapped", [(0, True), (1, True), (0, False), (1, False)])
def test_pack_head_against_compiled_reference(dtype, mapped):
    ref = O.ref_data_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rng = np.random.default_rng(12 + dtype)
    src = rng.integers(0, 65536, (40, 16), dtype=np.uint32).astype(np.uint16)
    mapping = rng.integers(0, 40, 23).astype(np.int32) if mapped else None
    want = _ref_compose_pack(ref, src, dtype, mapping)
    assert np.array_equal(O.pack_head(src, dtype, mapping).reshape(-1), want)


def test_load_vocab_map(tmp_path):
    from pumice_amd import lmhead as L
    from pumice_amd import sampler as S
    m = np.random.default_rng(13).permutation(5000)[:1000].astype(np.int32)
    p = tmp_path / "mapping.npy"
    np.save(p, m)
    assert np.array_equal(L.load_vocab_map(p, 1000), m)
    with pytest.raises(S.PssError):
        L.load_vocab_map(p, 999)                      # length mismatch
    np.save(tmp_path / "i8.npy", m.astype(np.int64))
    with pytest.raises(S.PssError):
        L.load_vocab_map(tmp_path / "i8.npy", 1000)   # not int32
    with open(tmp_path / "v2.npy", "wb") as f:
        np.lib.format.write_array(f, m, version=(2, 0))
    with pytest.raises(S.PssError):
        L.load_vocab_map(tmp_path / "v2.npy", 1000)   # only version 1, as the reference
    (tmp_path / "bad.npy").write_bytes(b"NOTNPY" + bytes(200))
    with pytest.raises(S.PssError):
        L.load_vocab_map(tmp_path / "bad.npy", 1000)
    with pytest.raises(S.PssError):
        L.load_vocab_map(tmp_path / "missing.npy", 1000)


def test_reference_mapping_file():
    path = "/root/reference/pruned-vocab/mapping.npy"
    if not os.path.exists(path):
        pytest.skip("reference checkout absent")
    from pumice_amd import lmhead as L
    m = L.load_vocab_map(path, 102400)
    want = np.load(path, allow_pickle=False)
    assert want.dtype == np.int32 and np.array_equal(m, want)
    assert m.min() >= 0 and m.max() < 248320 and np.unique(m).size == m.size
