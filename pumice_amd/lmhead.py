"""ctypes binding of the gfx950 LM head (include/pumice_lmhead.h): RMSNorm +
fp16 GEMV over the block-transposed head into logits (plh_logits, the
LMHead-GEMV-Q16 operation of src/generate.c:536-538) and the fused greedy form
writing the sampler's token state (plh_greedy, LMHead-GEMV-ArgMax-Q16 +
ArgMax-Reduce mode 0, src/generate.c:540-546)."""
import ctypes

import numpy as np

from . import sampler as S

TILE = 64
SLICES = 4
MAX_K = 65536

SRC_BF16, SRC_FP16 = 0, 1

EXPORTS = ["plh_create", "plh_destroy", "plh_logits", "plh_greedy", "plh_transpose_block16", "plh_stream",
           "plh_load_vocab_map", "plh_pack_head"]

_bound = False


def lib():
    global _bound
    L = S.lib()
    if not _bound:
        P, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
        L.plh_create.argtypes = [ctypes.POINTER(P), P, P, u32, u32, u32, P]
        L.plh_destroy.argtypes = [P]
        L.plh_logits.argtypes = [P, P, u64, u32, P, u64]
        L.plh_greedy.argtypes = [P, P, P, u64, u32, u32, u32]
        L.plh_transpose_block16.argtypes = [P, P, u32, u32]
        L.plh_stream.argtypes = [P]
        L.plh_stream.restype = P
        L.plh_load_vocab_map.argtypes = [ctypes.c_char_p, u32, P]
        L.plh_pack_head.argtypes = [P, u32, u32, u32, P, u32, P, P]
        for n in ("plh_create", "plh_destroy", "plh_logits", "plh_greedy", "plh_transpose_block16",
                  "plh_load_vocab_map", "plh_pack_head"):
            getattr(L, n).restype = i32
        _bound = True
    return L


def transpose_block16(w_kv):
    """Row-major fp16 [K][V] (as uint16 bits) -> block-transposed [K/8][V][8]
    through plh_transpose_block16 (src/data.c:305-331, QUANT_FP16)."""
    w = np.ascontiguousarray(w_kv, dtype=np.uint16)
    K, V = w.shape
    out = np.empty((K // 8, V, 8), np.uint16)
    S._ok(lib().plh_transpose_block16(w.ctypes.data, out.ctypes.data, K, V), "plh_transpose_block16")
    return out


def load_vocab_map(path, expected):
    """plh_load_vocab_map: pruned-vocab/mapping.npy -> int32[expected]."""
    out = np.zeros(int(expected), np.int32)
    S._ok(lib().plh_load_vocab_map(str(path).encode(), int(expected), out.ctypes.data), "plh_load_vocab_map")
    return out


def pack_head(src_ptr, src_dtype, src_rows, K, mapping, V, w_bt_ptr, stream=None):
    """plh_pack_head: device lm_head rows -> device block-transposed fp16 head."""
    m = None if mapping is None else np.ascontiguousarray(mapping, np.int32)
    S._ok(lib().plh_pack_head(src_ptr, src_dtype, src_rows, K, None if m is None else m.ctypes.data, V,
                              w_bt_ptr, stream), "plh_pack_head")


class LMHead:
    """The head over device-resident block-transposed fp16 weights and fp32 gamma."""

    def __init__(self, weight_ptr, gamma_ptr, K, V, max_rows, stream=None):
        self.K, self.V, self.max_rows = int(K), int(V), int(max_rows)
        h = ctypes.c_void_p()
        S._ok(lib().plh_create(ctypes.byref(h), weight_ptr, gamma_ptr, self.K, self.V, self.max_rows, stream),
              "plh_create")
        self.handle = h.value
        self.stream = lib().plh_stream(self.handle)

    def close(self):
        if self.handle:
            st = lib().plh_destroy(self.handle)
            self.handle = None
            S._ok(st, "plh_destroy")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            if self.handle:
                lib().plh_destroy(self.handle)
        except Exception:
            pass

    def logits(self, x_ptr, x_stride, rows, logits_ptr, logits_stride):
        S._ok(lib().plh_logits(self.handle, x_ptr, x_stride, rows, logits_ptr, logits_stride), "plh_logits")

    def greedy(self, sampler, x_ptr, x_stride, rows, do_increment=1, pass_idx=0):
        S._ok(lib().plh_greedy(self.handle, sampler.handle, x_ptr, x_stride, rows, do_increment, pass_idx),
              "plh_greedy")
