"""CPU oracle for the sampler path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker (or the timed CPU baseline).  The
product package (pumice_amd) never imports it.

Thin ctypes view of oracle/libpss_oracle.so (built by `make -C oracle`):
  O1 `o1_row` / `o1_batch`   exact build contract (sort-based restatement)
  O2 `o2_shader_row`         shader/Utility/ArgMax-Reduce.comp mode 1, literally
  O3 `o3_sampler_ref`        src/validation.c:4974-5092 (fp64 reference oracle)
  greedy / greedy_two_stage  ArgMax-Reduce.comp:135-167 + LMHead-GEMV-ArgMax-Q16.comp:75-96
  get_data                   src/data.c:8-28
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpss_oracle.so")
REF_DATA_PATH = os.path.join(HERE, "_ref", "libref_data.so")

MAX_PEN = 1024
SENTINEL = 0xFFFFFFFF

SAMPLE_PARAMS = np.dtype(
    [
        ("temperature", "<f4"),
        ("repPenalty", "<f4"),
        ("penaltyLength", "<u4"),
        ("topK", "<u4"),
        ("topP", "<f4"),
        ("minP", "<f4"),
        ("presencePenalty", "<f4"),
    ]
)
ROW_INFO = np.dtype(
    [
        ("token", "<u4"),
        ("kept_count", "<u4"),
        ("tau_key", "<u4"),
        ("tmax_key", "<u4"),
        ("z_kept", "<u8"),
        ("z_topk", "<u8"),
        ("target", "<u8"),
        ("u24", "<u4"),
        ("flags", "<u4"),
    ]
)
assert SAMPLE_PARAMS.itemsize == 28 and ROW_INFO.itemsize == 48

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle not built: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        u32, u64, f32, i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_int
        L.oracle_o1_row.restype = u32
        L.oracle_o1_row.argtypes = [P, u32, P, P, u32, u32, u32, u32, P, P, P, P, P]
        L.oracle_o1_batch.restype = None
        L.oracle_o1_batch.argtypes = [P, u32, u64, u32, u32, P, P, P, P, P, u32, u32, u32, P, P, i32]
        L.oracle_o1_batch_pinned.restype = None
        L.oracle_o1_batch_pinned.argtypes = [P, u32, u64, u32, u32, P, P, P, P, P, u32, u32, u32, P, i32, P]
        L.oracle_o3_batch_pinned.restype = None
        L.oracle_o3_batch_pinned.argtypes = [P, u64, u32, u32, P, P, P, P, P, i32, P]
        L.oracle_o2_shader_row.restype = u32
        L.oracle_o2_shader_row.argtypes = [P, u32, P, P, P, P, u32, P]
        L.oracle_o3_sampler_ref.restype = u32
        L.oracle_o3_sampler_ref.argtypes = [P, i32, P, P, P, P, u32, ctypes.c_double, P]
        L.oracle_greedy_row.restype = u32
        L.oracle_greedy_row.argtypes = [P, u32]
        L.oracle_greedy_two_stage.restype = u32
        L.oracle_greedy_two_stage.argtypes = [P, u32]
        L.oracle_get_pseudo_random.restype = f32
        L.oracle_get_pseudo_random.argtypes = [i32, i32, i32]
        L.oracle_get_data.restype = None
        L.oracle_get_data.argtypes = [i32, i32, i32, P]
        L.oracle_exp_scan.restype = u64
        L.oracle_exp_scan.argtypes = [f32, f32, u32, P, P]
        L.oracle_pss_exp.restype = f32
        L.oracle_pss_exp.argtypes = [f32]
        L.oracle_exp_many.restype = None
        L.oracle_exp_many.argtypes = [P, P, u64]
        L.oracle_prob_many.restype = None
        L.oracle_prob_many.argtypes = [P, f32, P, u64]
        L.oracle_philox4x32_10.restype = None
        L.oracle_philox4x32_10.argtypes = [P, P, P]
        L.oracle_xorshift32.restype = u32
        L.oracle_xorshift32.argtypes = [u32]
        L.oracle_topp_need.restype = u64
        L.oracle_topp_need.argtypes = [f32, u64]
        L.oracle_draw_target.restype = u64
        L.oracle_draw_target.argtypes = [u32, u64]
        L.oracle_key.restype = u32
        L.oracle_key.argtypes = [f32]
        L.oracle_unkey.restype = f32
        L.oracle_unkey.argtypes = [u32]
        L.oracle_canon.restype = f32
        L.oracle_canon.argtypes = [f32]
        L.oracle_fixq.restype = u64
        L.oracle_fixq.argtypes = [f32]
        L.oracle_h2f.restype = f32
        L.oracle_h2f.argtypes = [ctypes.c_uint16]
        L.oracle_o1_score_row.restype = f32
        L.oracle_o1_score_row.argtypes = [P, u32, u32, P, P]
        L.oracle_log64.restype = ctypes.c_double
        L.oracle_log64.argtypes = [ctypes.c_double]
        L.oracle_float_to_fp16_many.restype = None
        L.oracle_float_to_fp16_many.argtypes = [P, P, u64]
        L.oracle_fp16_to_float_many.restype = None
        L.oracle_fp16_to_float_many.argtypes = [P, P, u64]
        L.oracle_get_data_fp16.restype = None
        L.oracle_get_data_fp16.argtypes = [i32, i32, i32, P]
        L.oracle_transpose_block16_fp16.restype = None
        L.oracle_transpose_block16_fp16.argtypes = [P, P, u32, u32]
        L.oracle_float_to_bf16_many.restype = None
        L.oracle_float_to_bf16_many.argtypes = [P, P, u64]
        L.oracle_pack_head.restype = None
        L.oracle_pack_head.argtypes = [P, u32, u32, P, u32, P]
        L.oracle_lmhead_norm.restype = f32
        L.oracle_lmhead_norm.argtypes = [P, P, u32, P]
        L.oracle_lmhead_logits.restype = None
        L.oracle_lmhead_logits.argtypes = [P, P, u32, u32, u32, P]
        L.oracle_lmhead_logits64.restype = None
        L.oracle_lmhead_logits64.argtypes = [P, P, u32, u32, P, P]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def make_params(temperature=1.0, repPenalty=1.0, penaltyLength=0, topK=0, topP=1.0, minP=0.0,
                presencePenalty=0.0, rows=None):
    """One sample_params record (or `rows` copies)."""
    rec = np.zeros(1 if rows is None else rows, dtype=SAMPLE_PARAMS)
    rec["temperature"] = temperature
    rec["repPenalty"] = repPenalty
    rec["penaltyLength"] = penaltyLength
    rec["topK"] = topK
    rec["topP"] = topP
    rec["minP"] = minP
    rec["presencePenalty"] = presencePenalty
    return rec


def new_history(rows=None, fill=SENTINEL):
    shape = (MAX_PEN,) if rows is None else (rows, MAX_PEN)
    return np.full(shape, fill, dtype=np.uint32)


class RowState:
    """Mutable per-row state mirroring the GPU sampler's (history ring, position, rng, step)."""

    def __init__(self, history=None, position=0, rng=0, step=0):
        self.history = new_history() if history is None else np.ascontiguousarray(history, np.uint32).copy()
        assert self.history.shape == (MAX_PEN,)
        self.position, self.rng, self.step = int(position), int(rng), int(step)

    def copy(self):
        return RowState(self.history, self.position, self.rng, self.step)


class _CState(ctypes.Structure):
    _fields_ = [("history", ctypes.c_void_p), ("position", ctypes.c_uint32),
                ("rng", ctypes.c_uint32), ("step", ctypes.c_uint32)]


def o1_row(logits, params, state, row=0, mode=1, rng_mode=0, do_increment=1, want_kept=True,
           want_p=False, want_probs=False, want_probs64=False):
    """O1 on one fp32 row; mutates `state`. Returns dict(token, info, kept, p, probs, probs64)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    V = x.size
    prm = np.ascontiguousarray(params, dtype=SAMPLE_PARAMS).reshape(-1)[:1].copy()
    cs = _CState(state.history.ctypes.data, state.position, state.rng, state.step)
    info = np.zeros(1, ROW_INFO)
    kept = np.zeros(V, np.uint8) if want_kept else None
    p = np.zeros(V, np.float32) if want_p else None
    probs = np.zeros(V, np.float32) if want_probs else None
    probs64 = np.zeros(V, np.float64) if want_probs64 else None
    tok = lib().oracle_o1_row(_ptr(x), V, _ptr(prm), ctypes.addressof(cs), row, mode, rng_mode,
                              do_increment, _ptr(info), _ptr(kept), _ptr(p), _ptr(probs), _ptr(probs64))
    state.position, state.rng, state.step = cs.position, cs.rng, cs.step
    return dict(token=int(tok), info=info[0], kept=kept, p=p, probs=probs, probs64=probs64)


def o1_batch(logits, params, history, position, rng, step, mode=1, rng_mode=0, do_increment=1,
             threads=1, dtype=None):
    """O1 over rows; logits [rows, V] float32 or float16.  State arrays updated in place."""
    x = np.ascontiguousarray(logits)
    rows, V = x.shape
    if dtype is None:
        dtype = 1 if x.dtype == np.float16 else 0
    if dtype == 0:
        x = x.astype(np.float32, copy=False)
    prm = np.ascontiguousarray(params, dtype=SAMPLE_PARAMS)
    assert prm.shape == (rows,) and history.shape == (rows, MAX_PEN)
    for a in (history, position, rng, step):
        assert a.dtype == np.uint32 and a.flags.c_contiguous
    tokens = np.zeros(rows, np.uint32)
    infos = np.zeros(rows, ROW_INFO)
    lib().oracle_o1_batch(_ptr(x), dtype, V, rows, V, _ptr(prm), _ptr(history), _ptr(position),
                          _ptr(rng), _ptr(step), mode, rng_mode, do_increment, _ptr(tokens),
                          _ptr(infos), int(threads))
    return tokens, infos


def batch_pinned(kind, logits, params, history, position, rng, step, cpus):
    """The CPU baseline's batch: O1 ("o1") or O3 ("o3", fp32 rows) over all
    rows, one thread per entry of `cpus`, thread i pinned to cpus[i].  State
    arrays updated in place; returns the tokens."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = x.shape
    prm = np.ascontiguousarray(params, dtype=SAMPLE_PARAMS)
    cp = np.ascontiguousarray(cpus, dtype=np.int32)
    tokens = np.zeros(rows, np.uint32)
    if kind == "o1":
        lib().oracle_o1_batch_pinned(_ptr(x), 0, V, rows, V, _ptr(prm), _ptr(history), _ptr(position),
                                     _ptr(rng), _ptr(step), 1, 0, 1, _ptr(tokens), cp.size, _ptr(cp))
    else:
        lib().oracle_o3_batch_pinned(_ptr(x), V, rows, V, _ptr(prm), _ptr(history), _ptr(position),
                                     _ptr(rng), _ptr(tokens), cp.size, _ptr(cp))
    return tokens


def o1_score_row(logits, target):
    """Scoring mode on one row (fp32 values; fp16 rows widen exactly first).
    Returns (nll as float32 bits, Zq, key of the row maximum)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    zq = np.zeros(1, np.uint64)
    gk = np.zeros(1, np.uint32)
    nll = lib().oracle_o1_score_row(_ptr(x), x.size, int(target), _ptr(zq), _ptr(gk))
    return int(np.float32(nll).view(np.uint32)), int(zq[0]), int(gk[0])


def log64(x):
    return lib().oracle_log64(float(x))


def o2_shader_row(logits, params, history, position, rng, do_increment=1):
    """O2: returns (token, final p-space threshold, mutated logits, position, rng)."""
    x = np.ascontiguousarray(logits, dtype=np.float32).copy()
    prm = np.ascontiguousarray(params, dtype=SAMPLE_PARAMS).reshape(-1)[:1].copy()
    pos = np.array([position], np.uint32)
    r = np.array([rng], np.uint32)
    thr = np.zeros(1, np.float32)
    tok = lib().oracle_o2_shader_row(_ptr(x), x.size, _ptr(prm), _ptr(history), _ptr(pos), _ptr(r),
                                     do_increment, _ptr(thr))
    return int(tok), float(thr[0]), x, int(pos[0]), int(r[0])


def o3_sampler_ref(logits, params, history, position, rng, accept_tok=SENTINEL, tol=5e-4):
    """O3: returns (token, tolerance_used, mutated logits, position, rng)."""
    x = np.ascontiguousarray(logits, dtype=np.float32).copy()
    prm = np.ascontiguousarray(params, dtype=SAMPLE_PARAMS).reshape(-1)[:1].copy()
    pos = np.array([position], np.uint32)
    r = np.array([rng], np.uint32)
    tol_out = np.zeros(1, np.int32)
    tok = lib().oracle_o3_sampler_ref(_ptr(x), x.size, _ptr(prm), _ptr(history), _ptr(pos), _ptr(r),
                                      accept_tok, tol, _ptr(tol_out))
    return int(tok), bool(tol_out[0]), x, int(pos[0]), int(r[0])


def greedy(logits):
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().oracle_greedy_row(_ptr(x), x.size))


def greedy_two_stage(logits):
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().oracle_greedy_two_stage(_ptr(x), x.size))


def get_data(seed, M, N):
    out = np.zeros((M, N), np.float32)
    lib().oracle_get_data(seed, M, N, _ptr(out))
    return out


def float_to_fp16(f):
    """src/data.c:30-52 (truncating) over an array; returns uint16 bits."""
    f = np.ascontiguousarray(f, np.float32)
    h = np.zeros(f.shape, np.uint16)
    lib().oracle_float_to_fp16_many(_ptr(f), _ptr(h), f.size)
    return h


def fp16_to_float(h):
    h = np.ascontiguousarray(h, np.uint16)
    f = np.zeros(h.shape, np.float32)
    lib().oracle_fp16_to_float_many(_ptr(h), _ptr(f), h.size)
    return f


def get_data_fp16(seed, M, N):
    """src/data.c:83-93 getDataFP16: uint16 bits [M][N]."""
    out = np.zeros((M, N), np.uint16)
    lib().oracle_get_data_fp16(seed, M, N, _ptr(out))
    return out


def transpose_block16(w_kv):
    """src/data.c:305-331 (FP16): [K][V] -> [K/8][V][8]."""
    w = np.ascontiguousarray(w_kv, np.uint16)
    K, V = w.shape
    out = np.zeros((K // 8, V, 8), np.uint16)
    lib().oracle_transpose_block16_fp16(_ptr(w), _ptr(out), K, V)
    return out


def float_to_bf16(f):
    """src/data.c:194-200 over an array; returns uint16 bits."""
    f = np.ascontiguousarray(f, np.float32)
    b = np.zeros(f.shape, np.uint16)
    lib().oracle_float_to_bf16_many(_ptr(f), _ptr(b), f.size)
    return b


def pack_head(src, src_dtype, mapping=None):
    """The reference's load-time fp16 head (gather, conversions, transpose)
    from lm_head rows src[src_rows][K] (uint16 bits; src_dtype 0 bf16, 1 fp16)
    -> [K/8][V][8]."""
    src = np.ascontiguousarray(src, np.uint16)
    K = src.shape[1]
    if mapping is None:
        V, mp = src.shape[0], None
    else:
        m = np.ascontiguousarray(mapping, np.int32)
        V, mp = m.size, _ptr(m)
    out = np.zeros((K // 8, V, 8), np.uint16)
    lib().oracle_pack_head(_ptr(src), src_dtype, K, mp, V, _ptr(out))
    return out


def lmhead_norm(x, gamma):
    """RMSNorm of LMHead-GEMV-Q16.comp:34-58 in the GPU's order: (inv_rms, a)."""
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    a = np.zeros(x.size, np.float32)
    inv = lib().oracle_lmhead_norm(_ptr(x), _ptr(g), x.size, _ptr(a))
    return float(np.float32(inv)), a


def lmhead_logits(a, w_bt, slices=4):
    """GEMV of LMHead-GEMV-Q16.comp:60-70 in the GPU's K-slice order (fp32)."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w_bt, np.uint16)
    KB, V, _ = w.shape
    out = np.zeros(V, np.float32)
    lib().oracle_lmhead_logits(_ptr(a), _ptr(w), 8 * KB, V, slices, _ptr(out))
    return out


def lmhead_logits64(a, w_bt):
    """The same GEMV in binary64, with sum |a w| per column."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w_bt, np.uint16)
    KB, V, _ = w.shape
    out = np.zeros(V, np.float64)
    absdot = np.zeros(V, np.float64)
    lib().oracle_lmhead_logits64(_ptr(a), _ptr(w), 8 * KB, V, _ptr(out), _ptr(absdot))
    return out, absdot


def exp_many(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    lib().oracle_exp_many(_ptr(x), _ptr(y), x.size)
    return y


def prob_many(t, tmax):
    """pss_prob(t, tmax) elementwise: exp(t - tmax) of canonical fp32 values."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    y = np.zeros_like(t)
    lib().oracle_prob_many(_ptr(t), float(np.float32(tmax)), _ptr(y), t.size)
    return y


def exp_scan(lo, hi, acc_stride=1):
    mu = np.zeros(1, np.float64)
    wx = np.zeros(1, np.float32)
    v = lib().oracle_exp_scan(lo, hi, acc_stride, _ptr(mu), _ptr(wx))
    return int(v), float(mu[0]), float(wx[0])


def philox4x32_10(ctr, key):
    c = np.array(ctr, np.uint32)
    k = np.array(key, np.uint32)
    out = np.zeros(4, np.uint32)
    lib().oracle_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return [int(v) for v in out]


def xorshift32(x):
    return int(lib().oracle_xorshift32(x))


def topp_need(topP, zk):
    return int(lib().oracle_topp_need(topP, zk))


def draw_target(u24, z):
    return int(lib().oracle_draw_target(u24, z))


def key(t):
    return int(lib().oracle_key(t))


def keys(t):
    """Vectorised order-preserving key of canonical float32 values."""
    b = np.ascontiguousarray(t, np.float32).view(np.uint32)
    return np.where(b & 0x80000000, ~b, b | 0x80000000).astype(np.uint32)


def fixq(p):
    return int(lib().oracle_fixq(p))


def ref_data_lib():
    """The reference's own src/data.c built by oracle/Makefile (None if absent)."""
    if not os.path.exists(REF_DATA_PATH):
        return None
    L = ctypes.CDLL(REF_DATA_PATH)
    L.get_pseudo_random.restype = ctypes.c_float
    L.get_pseudo_random.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return L
