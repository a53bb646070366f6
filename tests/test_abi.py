"""C ABI checks that need no GPU: the library loads, exports every entry point
include/pumice_sampler.h declares, keeps sample_params byte-identical to the
reference (include/state.h:8-16), and its pure host helpers behave."""
import ctypes
import os
import re

import numpy as np
import pytest

from pumice_amd import sampler as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_entry_points():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(ROOT, "include", fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(pss_\w+|pgl_\w+|plh_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    L = S.lib()
    names = declared_entry_points()
    assert "pss_create" in names and "pss_enqueue" in names and "plh_logits" in names
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_sample_params_layout_matches_reference():
    # include/state.h:8-16: float temperature, float repPenalty, uint32_t penaltyLength,
    # uint32_t topK, float topP, float minP, float presencePenalty  -> 28 bytes
    expect = [("temperature", 0, "f"), ("repPenalty", 4, "f"), ("penaltyLength", 8, "u"),
              ("topK", 12, "u"), ("topP", 16, "f"), ("minP", 20, "f"), ("presencePenalty", 24, "f")]
    assert ctypes.sizeof(S.CSampleParams) == 28 and S.SAMPLE_PARAMS.itemsize == 28
    for name, off, kind in expect:
        assert getattr(S.CSampleParams, name).offset == off
        assert S.SAMPLE_PARAMS.fields[name][1] == off
        assert S.SAMPLE_PARAMS.fields[name][0].kind == kind
    # the wire header of the stdin server is <ffIIfffI (src/compute.c:103-112): params + seed
    import struct
    p = S.make_params(1, temperature=0.6, repPenalty=1.05, penaltyLength=64, topK=20, topP=0.95)
    assert p.tobytes() == struct.pack("<ffIIfff", 0.6, 1.05, 64, 20, 0.95, 0.0, 0.0)


def test_row_info_layout():
    assert S.ROW_INFO.itemsize == 48
    assert S.ROW_INFO.fields["z_kept"][1] == 16 and S.ROW_INFO.fields["u24"][1] == 40


def test_sanitize_request_matches_stdin_server():
    # src/compute.c:113-114
    p = S.make_params(1, temperature=0.7, penaltyLength=5000)[0]
    q, seed = S.sanitize_request(p, 0)
    assert q["penaltyLength"] == 1024 and seed == 1
    q, seed = S.sanitize_request(S.make_params(1, penaltyLength=64)[0], 77)
    assert q["penaltyLength"] == 64 and seed == 77


def test_host_helpers():
    assert S.mask_words(1) == 1 and S.mask_words(32) == 1 and S.mask_words(33) == 2
    assert S.mask_words(102400) == 3200 and S.mask_words(248320) == 7760
    L = S.lib()
    for st, txt in S.STATUS.items():
        assert L.pss_status_string(st).decode() == txt


def test_null_handles_rejected_without_gpu():
    L = S.lib()
    assert L.pss_destroy(None) == 1
    assert L.pss_set_params(None, 0, 1, None, None) == 1
    assert L.pss_enqueue(None, None, 0, 1, 1, 1, 1, 0, 0) == 1
    assert L.pss_read_results(None, 1, None, None) == 1
    h = ctypes.c_void_p()
    assert L.pss_create(None, 100, 1, None) == 1
    assert L.pss_create(ctypes.byref(h), 0, 1, None) == 1
    assert L.pss_create(ctypes.byref(h), S.MAX_VOCAB + 1, 1, None) == 4


def test_noalloc_rejects_more_rows_than_its_workspace_without_gpu():
    # checked on the host before any device call (the pointers are never used)
    L = S.lib()
    sp = S.CStatePtrs(*([16] * len(S.CStatePtrs._fields_)))
    args = lambda rows: (16, ctypes.byref(sp), 1000, 16, S.DTYPE_F32, 1000, rows, S.MODE_SAMPLE, 1, 0,
                         S.RNG_XORSHIFT32, 0, 0, None, None)
    assert L.pss_enqueue_noalloc(*args(S.NOALLOC_MAX_ROWS + 1)) == 1
    assert L.pss_enqueue_noalloc(*args(0)) == 1
    assert L.pss_enqueue_noalloc(None, ctypes.byref(sp), 1000, 16, 0, 1000, 1, 1, 1, 0, 0, 0, 0, None, None) == 1
