"""Python mirror of the sampler C ABI (include/pumice_sampler.h) over ctypes.

Names and argument meaning follow the reference's host interface for this
path: `set_params` = generatorSetSampling (src/generate.c:1411-1430),
`reset_history` = resetGenerator's ring reset (src/generate.c:1238-1252),
`set_position` = stateSetPosition (src/generate.c:993), `enqueue` = the
ArgMax-Reduce operation of buildLmHead (src/generate.c:545-547), `read_results`
= readBuffer(st->result) (src/generate.c:1131).  Errors raise PssError carrying
the C status code.

There is no CPU fallback: loading fails loudly when the HIP library is missing.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpumice_sampler.so")

MAX_PENALTY_LEN = 1024
RESULT_SLOTS = 4
MAX_VOCAB = 262144
SENTINEL = 0xFFFFFFFF

DTYPE_F32, DTYPE_F16 = 0, 1
MODE_GREEDY, MODE_SAMPLE, MODE_SCORE = 0, 1, 2
RNG_XORSHIFT32, RNG_PHILOX = 0, 1
INFO_GREEDY, INFO_FALLBACK, INFO_SCORE = 1, 2, 4
ENQ_GENERAL = 1
ENQ_SPLIT = 2
ENQ_FUSED = 4
ENQ_SMALL = 8
ENQ_GATED = 16
ENQ_RESIDENT = 32

STATUS = {0: "ok", 1: "invalid argument", 2: "allocation failed", 3: "HIP runtime error",
          4: "unsupported", 5: "no gfx950 device"}

# include/state.h:8-16, 28 bytes
SAMPLE_PARAMS = np.dtype(
    [("temperature", "<f4"), ("repPenalty", "<f4"), ("penaltyLength", "<u4"), ("topK", "<u4"),
     ("topP", "<f4"), ("minP", "<f4"), ("presencePenalty", "<f4")]
)
ROW_INFO = np.dtype(
    [("token", "<u4"), ("kept_count", "<u4"), ("tau_key", "<u4"), ("tmax_key", "<u4"),
     ("z_kept", "<u8"), ("z_topk", "<u8"), ("target", "<u8"), ("u24", "<u4"), ("flags", "<u4")]
)


class CSampleParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("repPenalty", ctypes.c_float),
                ("penaltyLength", ctypes.c_uint32), ("topK", ctypes.c_uint32),
                ("topP", ctypes.c_float), ("minP", ctypes.c_float),
                ("presencePenalty", ctypes.c_float)]


class CEnqueueOpts(ctypes.Structure):
    _fields_ = [("row_info", ctypes.c_void_p), ("kept_mask", ctypes.c_void_p),
                ("probs", ctypes.c_void_p), ("probs_stride", ctypes.c_uint64),
                ("host_tokens", ctypes.c_void_p), ("flags", ctypes.c_uint32),
                ("split_event", ctypes.c_void_p), ("gate_seq", ctypes.c_uint32), ("eos", ctypes.c_uint32)]


class CStatePtrs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("result", "token_ids", "position", "rng", "step", "history")]


EXPORTS = [
    "pss_create", "pss_destroy", "pss_set_params", "pss_reset_history", "pss_set_history",
    "pss_set_position", "pss_enqueue", "pss_enqueue_ex", "pss_read_results", "pss_read_state",
    "pss_get_state_ptrs", "pss_sanitize_request", "pss_stream", "pss_status_string",
    "pss_mask_words", "pss_set_score_targets", "pss_reset_gate", "pss_enqueue_noalloc",
    "pss_read_ceiling", "pss_read_ceiling_blocks",
]
NOALLOC_MAX_ROWS = 16


def enqueue_noalloc(params_ptr, state, vocab, logits_ptr, dtype, row_stride, rows, mode=MODE_SAMPLE,
                    do_increment=1, pass_idx=0, rng_mode=RNG_XORSHIFT32, max_topk=0, max_window=0,
                    row_info=None, stream=None):
    """pss_enqueue_noalloc: one step on caller-owned device buffers (state: a
    dict of device pointers with the pss_state_ptrs fields)."""
    sp = CStatePtrs(*[state[n] for n, _ in CStatePtrs._fields_])
    o = CEnqueueOpts(row_info, None, None, 0, None, 0, None, 0, 0xFFFFFFFF) if row_info else None
    _ok(lib().pss_enqueue_noalloc(params_ptr, ctypes.byref(sp), vocab, logits_ptr, dtype, row_stride, rows,
                                  mode, do_increment, pass_idx, rng_mode, max_topk, max_window,
                                  None if o is None else ctypes.byref(o), stream), "pss_enqueue_noalloc")


class PssError(RuntimeError):
    def __init__(self, status, what):
        super().__init__(f"{what}: {STATUS.get(status, status)} (status {status})")
        self.status = status


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP sampler library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        P, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
        L.pss_create.argtypes = [ctypes.POINTER(P), u32, u32, P]
        L.pss_destroy.argtypes = [P]
        L.pss_set_params.argtypes = [P, u32, u32, P, P]
        L.pss_reset_history.argtypes = [P, u32, u32, u32]
        L.pss_set_history.argtypes = [P, u32, u32, P, u32]
        L.pss_set_position.argtypes = [P, u32, u32, P]
        L.pss_set_score_targets.argtypes = [P, u32, u32, u32, P]
        L.pss_reset_gate.argtypes = [P]
        L.pss_enqueue.argtypes = [P, P, u32, u64, u32, u32, u32, u32, u32]
        L.pss_enqueue_ex.argtypes = [P, P, u32, u64, u32, u32, u32, u32, u32, P]
        L.pss_read_results.argtypes = [P, u32, P, P]
        L.pss_read_state.argtypes = [P, u32, P, P, P, P]
        L.pss_get_state_ptrs.argtypes = [P, P]
        L.pss_read_ceiling.argtypes = [P, u64, P, P]
        L.pss_read_ceiling_blocks.argtypes = [u64]
        L.pss_read_ceiling_blocks.restype = u32
        L.pss_enqueue_noalloc.argtypes = [P, P, u32, P, u32, u64, u32, u32, u32, u32, u32, u32, u32, P, P]
        L.pss_sanitize_request.argtypes = [P, P]
        L.pss_stream.argtypes = [P]
        L.pss_stream.restype = P
        L.pss_status_string.argtypes = [i32]
        L.pss_status_string.restype = ctypes.c_char_p
        L.pss_mask_words.argtypes = [u32]
        L.pss_mask_words.restype = u32
        for n in EXPORTS:
            f = getattr(L, n)
            if f.restype is ctypes.c_int and n not in ("pss_stream", "pss_status_string", "pss_mask_words",
                                                       "pss_read_ceiling_blocks"):
                f.restype = i32
        _lib = L
    return _lib


def _ok(st, what):
    if st != 0:
        raise PssError(st, what)


def make_params(rows=1, **kw):
    """Array of sample_params with the reference's neutral defaults
    (src/addon.c:396-402: T 0, rep 1, penLen 0, topK 0, topP 1, minP 0, presence 0)."""
    p = np.zeros(rows, SAMPLE_PARAMS)
    p["repPenalty"] = 1.0
    p["topP"] = 1.0
    for k, v in kw.items():
        p[k] = v
    return p


def sanitize_request(params, seed):
    """src/compute.c:113-114: penaltyLength clamped to 1024, seed 0 -> 1."""
    c = CSampleParams(*[params[f] for f in SAMPLE_PARAMS.names])
    s = ctypes.c_uint32(seed)
    _ok(lib().pss_sanitize_request(ctypes.byref(c), ctypes.byref(s)), "pss_sanitize_request")
    out = np.zeros(1, SAMPLE_PARAMS)
    for f in SAMPLE_PARAMS.names:
        out[f] = getattr(c, f)
    return out[0], s.value


def mask_words(vocab):
    return int(lib().pss_mask_words(vocab))


class Sampler:
    """One sampler object: `vocab` ids, up to `max_rows` independent rows."""

    def __init__(self, vocab, max_rows, stream=None):
        self.vocab, self.max_rows = int(vocab), int(max_rows)
        h = ctypes.c_void_p()
        _ok(lib().pss_create(ctypes.byref(h), self.vocab, self.max_rows, stream), "pss_create")
        self.handle = h.value
        self.stream = lib().pss_stream(self.handle)

    def close(self):
        if self.handle:
            st = lib().pss_destroy(self.handle)
            self.handle = None
            _ok(st, "pss_destroy")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            if self.handle:
                lib().pss_destroy(self.handle)
        except Exception:
            pass

    def set_params(self, params, seeds=None, row0=0):
        p = np.ascontiguousarray(params, dtype=SAMPLE_PARAMS).reshape(-1)
        s = None if seeds is None else np.ascontiguousarray(seeds, dtype=np.uint32).reshape(-1)
        if s is not None and s.size != p.size:
            raise ValueError("seeds and params differ in length")
        _ok(lib().pss_set_params(self.handle, row0, p.size, p.ctypes.data,
                                 None if s is None else s.ctypes.data), "pss_set_params")

    def reset_gate(self):
        _ok(lib().pss_reset_gate(self.handle), "pss_reset_gate")

    def reset_history(self, fill=SENTINEL, row0=0, rows=None):
        rows = self.max_rows - row0 if rows is None else rows
        _ok(lib().pss_reset_history(self.handle, row0, rows, fill), "pss_reset_history")

    def set_history(self, hist, row0=0):
        h = np.ascontiguousarray(hist, dtype=np.uint32)
        if h.ndim == 1:
            h = h[None, :]
        _ok(lib().pss_set_history(self.handle, row0, h.shape[0], h.ctypes.data, h.shape[1]),
            "pss_set_history")

    def set_score_targets(self, ids, row0=0):
        """ids [rows][slots] (slots <= 4): the token scored by pass slot k of each row."""
        t = np.ascontiguousarray(ids, dtype=np.uint32)
        if t.ndim == 1:
            t = t[:, None]
        _ok(lib().pss_set_score_targets(self.handle, row0, t.shape[0], t.shape[1], t.ctypes.data),
            "pss_set_score_targets")

    def set_position(self, pos, row0=0):
        p = np.ascontiguousarray(pos, dtype=np.uint32).reshape(-1)
        _ok(lib().pss_set_position(self.handle, row0, p.size, p.ctypes.data), "pss_set_position")

    def enqueue(self, logits_ptr, dtype, row_stride, rows, mode=MODE_SAMPLE, do_increment=1,
                pass_idx=0, rng_mode=RNG_XORSHIFT32, row_info=None, kept_mask=None, probs=None,
                probs_stride=0, host_tokens=None, flags=0, split_event=None, gate_seq=0, eos=0xFFFFFFFF):
        """One step; logits_ptr and the optional outputs are device pointers (ints).
        split_event: a hipEvent_t recorded between the step's two kernels.
        gate_seq / eos: the decode-group sequence number and EOS id of an
        ENQ_GATED pass."""
        if (row_info is None and kept_mask is None and probs is None and host_tokens is None
                and not flags and split_event is None):
            st = lib().pss_enqueue(self.handle, logits_ptr, dtype, row_stride, rows, mode,
                                   do_increment, pass_idx, rng_mode)
        else:
            o = CEnqueueOpts(row_info, kept_mask, probs, probs_stride, host_tokens, flags, split_event,
                             gate_seq, eos)
            st = lib().pss_enqueue_ex(self.handle, logits_ptr, dtype, row_stride, rows, mode,
                                      do_increment, pass_idx, rng_mode, ctypes.byref(o))
        _ok(st, "pss_enqueue")

    def read_results(self, rows=None):
        rows = self.max_rows if rows is None else rows
        res = np.zeros((rows, RESULT_SLOTS), np.uint32)
        tok = np.zeros(rows, np.uint32)
        _ok(lib().pss_read_results(self.handle, rows, res.ctypes.data, tok.ctypes.data), "pss_read_results")
        return res, tok

    def read_state(self, rows=None):
        rows = self.max_rows if rows is None else rows
        hist = np.zeros((rows, MAX_PENALTY_LEN), np.uint32)
        pos = np.zeros(rows, np.uint32)
        rng = np.zeros(rows, np.uint32)
        step = np.zeros(rows, np.uint32)
        _ok(lib().pss_read_state(self.handle, rows, hist.ctypes.data, pos.ctypes.data,
                                 rng.ctypes.data, step.ctypes.data), "pss_read_state")
        return dict(history=hist, position=pos, rng=rng, step=step)

    def state_ptrs(self):
        p = CStatePtrs()
        _ok(lib().pss_get_state_ptrs(self.handle, ctypes.byref(p)), "pss_get_state_ptrs")
        return {n: getattr(p, n) for n, _ in CStatePtrs._fields_}
