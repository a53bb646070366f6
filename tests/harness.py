"""Shared helpers for the parity tests: one sampler step on the GPU through the
C ABI, the same step through the O1 oracle, and a field-by-field comparison."""
import numpy as np

import oracle as O
from pumice_amd import hip
from pumice_amd import sampler as S


def pack_mask(kept, words):
    """uint8 kept[V] -> little-endian bit words [words] (bit j of word j>>5)."""
    b = np.packbits(kept.astype(np.uint8), bitorder="little")
    out = np.zeros(words * 4, np.uint8)
    out[: b.size] = b
    return out.view(np.uint32)


class GpuRun:
    """A sampler plus device copies of a batch of logit rows."""

    def __init__(self, logits, params, seeds=None, history=None, position=None):
        self.logits = np.ascontiguousarray(logits)
        self.rows, self.V = self.logits.shape
        self.dtype = S.DTYPE_F16 if self.logits.dtype == np.float16 else S.DTYPE_F32
        self.s = S.Sampler(self.V, self.rows)
        self.dev = hip.DeviceBuffer.from_array(self.logits)
        self.mw = S.mask_words(self.V)
        self.s.set_params(params, seeds)
        if history is not None:
            self.s.set_history(history)
        if position is not None:
            self.s.set_position(position)

    def load(self, logits):
        logits = np.ascontiguousarray(logits, dtype=self.logits.dtype)
        assert logits.shape == (self.rows, self.V)
        self.logits = logits
        self.dev.upload(logits)

    def step(self, mode=S.MODE_SAMPLE, rng_mode=S.RNG_XORSHIFT32, do_increment=1, pass_idx=0,
             want_mask=True, want_probs=False, flags=0):
        info = hip.DeviceBuffer(self.rows * S.ROW_INFO.itemsize)
        mask = hip.DeviceBuffer(self.rows * self.mw * 4) if want_mask else None
        probs = hip.DeviceBuffer(self.rows * self.V * 4) if want_probs else None
        self.s.enqueue(self.dev.ptr, self.dtype, self.V, self.rows, mode, do_increment, pass_idx,
                       rng_mode, row_info=info.ptr, kept_mask=mask.ptr if mask else None,
                       probs=probs.ptr if probs else None, probs_stride=self.V if probs else 0,
                       flags=flags)
        res, tok = self.s.read_results(self.rows)
        out = dict(result=res, tokens=tok, info=info.download(S.ROW_INFO, self.rows))
        if mask:
            out["mask"] = mask.download(np.uint32, (self.rows, self.mw))
        if probs:
            out["probs"] = probs.download(np.float32, (self.rows, self.V))
        return out

    def state(self):
        return self.s.read_state(self.rows)

    def close(self):
        self.s.close()
        self.dev.free()


class OracleRun:
    """O1 with the same per-row state as the GPU sampler."""

    def __init__(self, rows, params, seeds=None, history=None, position=None):
        self.rows = rows
        self.params = np.ascontiguousarray(params, dtype=O.SAMPLE_PARAMS)
        self.states = []
        for r in range(rows):
            h = O.new_history() if history is None else np.asarray(history[r], np.uint32)
            self.states.append(O.RowState(h, 0 if position is None else int(position[r]),
                                          0 if seeds is None else int(seeds[r]), 0))

    def step(self, logits, mode=1, rng_mode=0, do_increment=1, want_kept=True, want_probs=False,
             want_probs64=False, want_p=False):
        x = np.asarray(logits)
        if x.dtype == np.float16:
            x = x.astype(np.float32)
        outs = []
        for r in range(self.rows):
            outs.append(O.o1_row(x[r], self.params[r], self.states[r], row=r, mode=mode,
                                 rng_mode=rng_mode, do_increment=do_increment, want_kept=want_kept,
                                 want_probs=want_probs, want_probs64=want_probs64, want_p=want_p))
        return outs


INFO_FIELDS = ("token", "kept_count", "tau_key", "tmax_key", "z_kept", "z_topk", "target", "u24", "flags")


def compare_step(g, outs, pass_idx=0, mw=None, check_probs=False, where=""):
    """Assert GPU step outputs equal the oracle's row by row (bit-exact)."""
    rows = len(outs)
    for r in range(rows):
        o = outs[r]
        gi = g["info"][r]
        for f in INFO_FIELDS:
            assert int(gi[f]) == int(o["info"][f]), (
                f"{where} row {r}: {f} gpu={int(gi[f])} oracle={int(o['info'][f])}")
        assert int(g["tokens"][r]) == o["token"], f"{where} row {r}: token_ids"
        assert int(g["result"][r, pass_idx]) == o["token"], f"{where} row {r}: result slot"
        if "mask" in g and o["kept"] is not None:
            exp = pack_mask(o["kept"], g["mask"].shape[1])
            bad = np.nonzero(g["mask"][r] != exp)[0]
            assert bad.size == 0, f"{where} row {r}: kept mask differs in {bad.size} words (first {bad[:4]})"
        if check_probs and "probs" in g:
            gp, op = g["probs"][r], o["probs"]
            assert np.array_equal(gp.view(np.uint32), op.view(np.uint32)), (
                f"{where} row {r}: probs differ at {np.nonzero(gp != op)[0][:5]}")


def compare_state(gst, ost, where=""):
    for r, st in enumerate(ost.states):
        assert int(gst["position"][r]) == st.position, f"{where} row {r}: position"
        assert int(gst["rng"][r]) == st.rng, f"{where} row {r}: rng"
        assert int(gst["step"][r]) == st.step, f"{where} row {r}: philox step"
        assert np.array_equal(gst["history"][r], st.history), f"{where} row {r}: history ring"
