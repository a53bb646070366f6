"""Write the golden fixtures under tests/golden/.

  get_data_777001.json  getData(777001, 1, 102400) bit patterns at 96 ids, as
                        produced by the reference's own src/data.c, compiled
                        from its source into oracle/_ref/ by oracle/Makefile.
  validator_o1.json     the reference validator's four cases x 3 chained draws
                        (src/validation.c:5094-5185): O1 token and diagnostics
                        per draw, the O3 (restated sampler_ref) token, and
                        the final position / history ring checksum.
  configs_o1.json       O1 tokens for small seeded instances of c1-c5.
  fp16_data.json        the reference's own src/data.c fp16 helpers (compiled
                        into oracle/_ref/): float_to_fp16 on 64 binary32 bit
                        patterns, getDataFP16(15001, 4096, 102400) at 64
                        (k, n) positions (the LM-head weights of the
                        validation run, src/validation.c:6174), and
                        transpose_block16(QUANT_FP16) of a 16 x 5 matrix,
                        float_to_bf16 on the same 64 patterns.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from pumice_amd import workloads as WL  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
INFO = ("token", "kept_count", "tau_key", "tmax_key", "z_kept", "z_topk", "target", "u24", "flags")


def get_data_fixture():
    ref = O.ref_data_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_data.so missing: run `make -C oracle` with the reference present")
    V = WL.V_PRUNED
    ids = sorted(set([0, 1, 2, 3, V - 1, V - 2] + list(np.random.default_rng(0).integers(0, V, 90))))
    bits = [int(np.float32(ref.get_pseudo_random(0, int(j), 777001)).view(np.uint32)) for j in ids]
    return {"seed": 777001, "M": 1, "N": V, "ids": [int(j) for j in ids], "bits": bits,
            "source": "reference src/data.c get_pseudo_random, compiled by oracle/Makefile"}


def validator_fixture():
    V = WL.V_PRUNED
    hist, pos0, cases, seeds = WL.validator_inputs(V)
    x = O.get_data(777001, 1, V)[0]
    st = O.RowState(hist, pos0, 0, 0)
    draws = []
    for c in range(4):
        st.rng = int(seeds[c])
        for d in range(3):
            h, p, r = st.history.copy(), st.position, st.rng
            o = O.o1_row(x, cases[c], st, want_p=True)
            t3, _, _, _, _ = O.o3_sampler_ref(x, cases[c], h.copy(), p, r)
            draws.append({"case": "ABCD"[c], "draw": d, "o1": {f: int(o["info"][f]) for f in INFO},
                          "o3_token": t3})
            x = o["p"]
    return {"V": V, "pos0": pos0, "draws": draws, "final_position": st.position,
            "final_history_sum": int(st.history.astype(np.uint64).sum())}


def configs_fixture():
    out = {}
    w, spikes = WL.c1(seed=0)
    out["c1_greedy"] = O.greedy(w.logits[0])
    st = O.RowState(w.history[0], 0, 0, 0)
    out["c1_sample"] = O.o1_row(w.logits[0], w.params[0], st)["token"]
    for name, w in [("c3", WL.c3(seed=21, rows=4)), ("c4", WL.c4(seed=22, rows=2)), ("c5", WL.c5(seed=23, rows=8))]:
        toks = []
        for r in range(w.rows):
            st = O.RowState(w.history[r], 0, int(w.seeds[r]), 0)
            toks.append(O.o1_row(w.logits[r].astype(np.float32), w.params[r], st, row=r)["token"])
        out[name] = toks
    w, xs = WL.c2(seed=24, rows=1, steps=8)
    st = O.RowState(w.history[0], 0, 99, 0)
    out["c2_chain"] = [O.o1_row(xs[k, 0], w.params[0], st)["token"] for k in range(8)]
    st = O.RowState(w.history[0], 0, 99, 0)
    out["c2_chain_philox"] = [O.o1_row(xs[k, 0], w.params[0], st, rng_mode=1)["token"] for k in range(8)]
    return out


def fp16_fixture():
    import ctypes
    ref = O.ref_data_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_data.so missing: run `make -C oracle` with the reference present")
    ref.float_to_fp16.restype = ctypes.c_uint16
    ref.float_to_fp16.argtypes = [ctypes.c_float]
    ref.getDataFP16.restype = ctypes.c_void_p
    ref.getDataFP16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    ref.float_to_bf16.restype = ctypes.c_uint16
    ref.float_to_bf16.argtypes = [ctypes.c_float]
    ref.transpose_block16.restype = None
    ref.transpose_block16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    libc = ctypes.CDLL(None)
    libc.free.argtypes = [ctypes.c_void_p]
    rng = np.random.default_rng(5)
    fixed = [0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 70000.0, 1e-5, 6.1035156e-05, 5.9604645e-08, 2.9e-08,
             1e-9, 0.1, -0.3333333, 3.14159265, np.inf, -np.inf, 1e30]
    f = np.array(fixed + list(rng.normal(0, 4, 30)) + list(rng.uniform(-1, 1, 16)), np.float32)
    fbits = f.view(np.uint32)
    hbits = [int(ref.float_to_fp16(float(v))) for v in f]
    K, V = 4096, 102400
    ptr = ref.getDataFP16(15001, K, V)
    data = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint16)), shape=(K * V,))
    pos = [(0, 0), (0, 1), (1, 0), (K - 1, V - 1), (K - 1, 0), (0, V - 1)] + \
        [(int(i), int(j)) for i, j in zip(rng.integers(0, K, 58), rng.integers(0, V, 58))]
    gvals = [int(data[i * V + j]) for i, j in pos]
    libc.free(ptr)
    w = rng.integers(0, 65536, (16, 5), dtype=np.uint16)
    out = np.zeros(16 * 5, np.uint16)
    ref.transpose_block16(w.ctypes.data, out.ctypes.data, 16, 5, 16)
    bbits = [int(ref.float_to_bf16(float(v))) for v in f]
    return {"float_to_fp16": {"in_bits": [int(b) for b in fbits], "out_bits": hbits},
            "float_to_bf16": {"in_bits": [int(b) for b in fbits], "out_bits": bbits},
            "get_data_fp16": {"seed": 15001, "M": K, "N": V, "pos": pos, "bits": gvals},
            "transpose_block16": {"K": 16, "V": 5, "in": w.reshape(-1).tolist(), "out": out.tolist()},
            "source": "reference src/data.c float_to_fp16 / float_to_bf16 / getDataFP16 / transpose_block16, "
                      "compiled by oracle/Makefile"}


def main():
    only = sys.argv[1:]
    for name, fn in [("get_data_777001.json", get_data_fixture), ("validator_o1.json", validator_fixture),
                     ("configs_o1.json", configs_fixture), ("fp16_data.json", fp16_fixture)]:
        if only and name not in only:
            continue
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(fn(), f, indent=1)
        print("wrote", name)


if __name__ == "__main__":
    main()
