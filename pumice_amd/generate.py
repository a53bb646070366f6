"""ctypes mirror of the C generate-loop call site (include/pumice_generate.h)."""
import ctypes

import numpy as np

from . import sampler as S

DECODE_GROUP = 4

LOGITS_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32)
EMIT_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32)


class CConfig(ctypes.Structure):
    _fields_ = [("max_new", ctypes.c_uint32), ("eos", ctypes.c_uint32), ("rows", ctypes.c_uint32),
                ("dtype", ctypes.c_uint32), ("row_stride", ctypes.c_uint64), ("mode", ctypes.c_uint32),
                ("rng_mode", ctypes.c_uint32), ("start_pos", ctypes.c_uint32)]


class CResult(ctypes.Structure):
    _fields_ = [("emitted", ctypes.c_uint32), ("finish_reason", ctypes.c_uint32),
                ("groups", ctypes.c_uint32), ("wall_us", ctypes.c_double)]


class CTable(ctypes.Structure):
    _fields_ = [("rows", ctypes.POINTER(ctypes.c_void_p)), ("count", ctypes.c_uint32)]


_bound = False


def _lib():
    global _bound
    L = S.lib()
    if not _bound:
        P, u32, u64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
        L.pgl_generate.argtypes = [P, P, P, P, P, P, P]
        L.pgl_generate.restype = ctypes.c_int
        L.pgl_generate_pinned.argtypes = [P, P, P, P, P, P, P, P, P]
        L.pgl_generate_pinned.restype = ctypes.c_int
        L.pgl_generate_pipelined.argtypes = [P, P, P, P, P, P, P, P, P]
        L.pgl_generate_pipelined.restype = ctypes.c_int
        L.pgl_score.argtypes = [P, P, P, u32, u64, P, u32, u32, P, P]
        L.pgl_score.restype = ctypes.c_int
        L.pgl_step_latency.argtypes = [P, P, P, u32, u64, u32, u32, P, P, P, P]
        L.pgl_step_latency.restype = ctypes.c_int
        L.pgl_table_logits.argtypes = [P, u32]
        L.pgl_table_logits.restype = P
        _bound = True
    return L


class LogitsTable:
    """Device logits rows cycled by position, read from C (pgl_table_logits)."""

    def __init__(self, dev_ptrs):
        self.ptrs = (ctypes.c_void_p * len(dev_ptrs))(*dev_ptrs)
        self.table = CTable(ctypes.cast(self.ptrs, ctypes.POINTER(ctypes.c_void_p)), len(dev_ptrs))
        self.fn = ctypes.cast(_lib().pgl_table_logits, ctypes.c_void_p).value

    @property
    def ctx(self):
        return ctypes.addressof(self.table)


def generate(sampler, table, max_new, rows=1, dtype=S.DTYPE_F32, row_stride=None, mode=S.MODE_SAMPLE,
             rng_mode=S.RNG_XORSHIFT32, eos=0xFFFFFFFF, start_pos=0, stop_after=None, pinned=None,
             pipelined=False):
    """pgl_generate; with `pinned` (a hip.PinnedBuffer of at least rows * 4
    u32) pgl_generate_pinned; with `pipelined` too (at least rows * 9 u32)
    pgl_generate_pipelined.  Returns (emitted tokens of row 0, result dict)."""
    out = []

    def _emit(ctx, tok):
        out.append(int(tok))
        return 1 if (stop_after is not None and len(out) >= stop_after) else 0

    emit = EMIT_FN(_emit)
    cfg = CConfig(max_new, eos, rows, dtype, row_stride or sampler.vocab, mode, rng_mode, start_pos)
    res = CResult()
    if pinned is None:
        if pipelined:
            raise ValueError("the pipelined loop needs a pinned buffer")
        name = "pgl_generate"
        st = _lib().pgl_generate(sampler.handle, ctypes.byref(cfg), table.fn, table.ctx,
                                 ctypes.cast(emit, ctypes.c_void_p), None, ctypes.byref(res))
    else:
        need = (9 if pipelined else 4) * rows * 4
        if pinned.nbytes < need:
            raise ValueError(f"pinned buffer smaller than {need} bytes")
        name = "pgl_generate_pipelined" if pipelined else "pgl_generate_pinned"
        st = getattr(_lib(), name)(sampler.handle, ctypes.byref(cfg), table.fn, table.ctx,
                                   ctypes.cast(emit, ctypes.c_void_p), None, pinned.dev_ptr, pinned.ptr,
                                   ctypes.byref(res))
    if st != 0:
        raise S.PssError(st, name)
    return out, dict(emitted=res.emitted, finish_reason=res.finish_reason, groups=res.groups,
                     wall_us=res.wall_us)


def step_latency(sampler, table, steps, pinned, dtype=S.DTYPE_F32, rng_mode=S.RNG_PHILOX):
    """pgl_step_latency; `pinned` is a hip.PinnedBuffer.  Returns (lat_us, tokens)."""
    lat = np.zeros(steps, np.float64)
    toks = np.zeros(steps, np.uint32)
    st = _lib().pgl_step_latency(sampler.handle, table.fn, table.ctx, dtype, sampler.vocab, rng_mode,
                                 steps, pinned.dev_ptr, pinned.ptr, lat.ctypes.data, toks.ctypes.data)
    if st != 0:
        raise S.PssError(st, "pgl_step_latency")
    return lat, toks


def score(sampler, table, ids, dtype=S.DTYPE_F32, row_stride=None, start_pos=0):
    """pgl_score over ids (row 0); returns (loss_sum, count)."""
    a = np.ascontiguousarray(ids, dtype=np.uint32)
    loss = ctypes.c_double()
    cnt = ctypes.c_uint64()
    st = _lib().pgl_score(sampler.handle, table.fn, table.ctx, dtype, row_stride or sampler.vocab,
                          a.ctypes.data, a.size, start_pos, ctypes.byref(loss), ctypes.byref(cnt))
    if st != 0:
        raise S.PssError(st, "pgl_score")
    return loss.value, cnt.value
