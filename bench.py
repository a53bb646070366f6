#!/usr/bin/env python3
"""Sampler benchmark on one MI355X: logits -> token, through the C ABI.

A "step" is one pss_enqueue over a batch of logit rows resident in HBM.

  headline  256 x 102,400 fp32 rows, rep 1.1 / presence 0.5 over a 64-id
            window, T 0.8, top-k 40, top-p 0.95, min-p 0.05  ->  `value` =
            sampled rows/s, plus algorithmic HBM GB/s and its roofline
            fraction.  Each step reads a different one of NBUF batches, so the
            working set (>= 600 MB) exceeds the 256 MB last-level cache and
            rows come from HBM.  One step is one launch of pss_res_kernel (the
            register-resident form; --fused / --split / --general force the
            other forms).
  latency   batch 1 (config c2; the small-batch form, pss_small_kernel):
            launch-to-token p50/p90 (host clock, token stored by the kernel
            into pinned host memory), per-step GPU time, and steady
            decode-group us/token through the C generate loops (per-group
            readback, pinned tokens, and pipelined: the next group queued
            before the current one is read).
  c3/c4/c5  the other batched configurations, rows/s and GB/s.
  lmhead    the LM head before the sampler (RMSNorm + fp16 GEMV over a
            4,096 x 102,400 block-transposed head): us per call and HBM GB/s
            for 1 and 4 rows, logits and fused-greedy forms.
  read_ceiling  pss_read_ceiling: the resident kernel's access pattern with
            nothing else, over the same bytes as one headline batch -- the
            achievable read rate the sampler's fraction is set beside.
  cpu_baseline  the O1 oracle (scalar C, sort-based) on the box's host cores,
            one pinned thread per allowed CPU (up to 16), over a bounded
            sample of the headline rows; one-thread and O3 (sampler_ref)
            lines beside it.

Prints ONE JSON line.  Algorithmic bytes per row = V*elem + 4*W + 44.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
TRAFFIC_MD = "sampler_traffic_by_config.md"
NBUF = 6


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pct(a, q):
    return float(np.percentile(np.asarray(a), q))


def copy_calibration(nbytes, reps=10):
    """Device-to-device copies of `nbytes` (one logits batch): a kernel of
    known traffic (nbytes read + nbytes written per dispatch) that scales the
    FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run."""
    from pumice_amd import hip

    src, dst = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    for _ in range(reps):
        hip.check(hip.rt().hipMemcpy(dst.ptr, src.ptr, nbytes, hip.hipMemcpyDeviceToDevice), "copy")
    hip.synchronize()
    src.free()
    dst.free()


def bench_batched(w, steps, warmup, flags=0):
    """rows/s and per-launch GPU time for workload `w` (rows x V).

    The default path is one kernel per step (pss_res_kernel); with
    S.ENQ_SPLIT it is two (pss_seg_kernel, then pss_fin_kernel) and the split
    event the library records between them times each one."""
    from pumice_amd import hip
    from pumice_amd import sampler as S

    dtype = S.DTYPE_F16 if w.logits.dtype == np.float16 else S.DTYPE_F32
    s = S.Sampler(w.V, w.rows)
    s.set_params(w.params, w.seeds)
    s.set_history(w.history)
    bufs = []
    for b in range(NBUF):
        bufs.append(hip.DeviceBuffer.from_array(np.roll(w.logits, 977 * b, axis=1)))
    stream = s.stream
    for i in range(warmup):
        s.enqueue(bufs[i % NBUF].ptr, dtype, w.V, w.rows, flags=flags)
    hip.stream_sync(stream)
    # timed region: exactly `steps` launches, synchronized on both sides, and
    # bracketed by HIP events on the sampler's stream (GPU time per launch,
    # back to back)
    ev0, ev1 = hip.Event(), hip.Event()
    hip.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        s.enqueue(bufs[i % NBUF].ptr, dtype, w.V, w.rows, flags=flags)
    ev1.record(stream)
    hip.stream_sync(stream)
    hip.synchronize()
    wall = time.perf_counter() - t0
    stream_ms = ev0.elapsed_ms(ev1) / steps
    # per-launch GPU time with HIP events on the sampler's stream around each
    # launch (and, split form, the event between its two kernels)
    n_ev = min(steps, 100)
    ev = [(hip.Event(), hip.Event(), hip.Event()) for _ in range(n_ev)]
    split = bool(flags & S.ENQ_SPLIT)
    for i in range(n_ev):
        ev[i][0].record(stream)
        s.enqueue(bufs[i % NBUF].ptr, dtype, w.V, w.rows, flags=flags,
                  split_event=ev[i][1].ptr if split else None)
        ev[i][2].record(stream)
    hip.stream_sync(stream)
    kt = [a.elapsed_ms(c) for a, b, c in ev]
    res, tok = s.read_results(w.rows)
    s.close()
    for b in bufs:
        b.free()
    bpr = w.bytes_per_row()
    k_ms = float(np.mean(kt))
    out = dict(rows=w.rows, V=w.V, dtype=str(w.logits.dtype), ms_per_step=wall * 1e3 / steps,
               rows_per_s=w.rows * steps / wall, stream_ms_per_launch=stream_ms,
               launch_ms_mean=k_ms, launch_ms_p50=pct(kt, 50),
               bytes_per_row=bpr, bytes_per_launch=bpr * w.rows,
               stream_gbps=bpr * w.rows / (stream_ms * 1e-3) / 1e9,
               launch_gbps=bpr * w.rows / (k_ms * 1e-3) / 1e9,
               wall_gbps=bpr * w.rows * steps / wall / 1e9)
    if split:
        seg = [a.elapsed_ms(b) for a, b, c in ev]
        out.update(seg_kernel_ms_mean=float(np.mean(seg)), fin_ms_mean=k_ms - float(np.mean(seg)))
    return out


def bench_latency(steps):
    """Batch-1 latency on config c2 with Philox (key 0, counter = step)."""
    from pumice_amd import generate as G
    from pumice_amd import hip
    from pumice_amd import sampler as S
    from pumice_amd import workloads as WL

    nrows = 64
    w, xs = WL.c2(seed=2, rows=1, steps=nrows)
    s = S.Sampler(w.V, 1)
    s.set_params(w.params, np.zeros(1, np.uint32))
    s.set_history(w.history)
    dev = [hip.DeviceBuffer.from_array(xs[k]) for k in range(nrows)]
    table = G.LogitsTable([d.ptr for d in dev])
    pinned = hip.PinnedBuffer(64)
    G.step_latency(s, table, 50, pinned)  # warm
    lat, toks = G.step_latency(s, table, steps, pinned)
    # per-step GPU time (events around each launch)
    stream = s.stream
    n_ev = min(steps, 200)
    ev = [(hip.Event(), hip.Event()) for _ in range(n_ev)]
    for i in range(n_ev):
        ev[i][0].record(stream)
        s.enqueue(dev[i % nrows].ptr, S.DTYPE_F32, w.V, 1, rng_mode=S.RNG_PHILOX)
        ev[i][1].record(stream)
    hip.stream_sync(stream)
    gpu_us = [a.elapsed_ms(b) * 1e3 for a, b in ev]
    # back-to-back steps (a decode loop whose next step is already queued):
    # events bracketing n_ev launches
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for i in range(n_ev):
        s.enqueue(dev[i % nrows].ptr, S.DTYPE_F32, w.V, 1, rng_mode=S.RNG_PHILOX)
    e1.record(stream)
    hip.stream_sync(stream)
    b2b_us = e0.elapsed_ms(e1) * 1e3 / n_ev
    # steady decode groups through the C generate loop: result slots copied
    # back per group (the reference's structure), then tokens through pinned
    # host memory; both from the same state, so the tokens must agree
    s.set_params(w.params, np.zeros(1, np.uint32))
    s.set_history(w.history)
    toks_gen, r = G.generate(s, table, steps, rows=1, rng_mode=S.RNG_PHILOX)
    s.set_params(w.params, np.zeros(1, np.uint32))
    s.set_history(w.history)
    toks_pin, rp = G.generate(s, table, steps, rows=1, rng_mode=S.RNG_PHILOX, pinned=pinned)
    # the pipelined loop: the next group is queued before the current one is
    # read (gated passes), so the GPU runs the steps back to back
    s.set_params(w.params, np.zeros(1, np.uint32))
    s.set_history(w.history)
    toks_pipe, rq = G.generate(s, table, steps, rows=1, rng_mode=S.RNG_PHILOX, pinned=pinned, pipelined=True)
    s.close()
    pinned.free()
    for d in dev:
        d.free()
    return dict(steps=steps, launch_to_token_us_p50=pct(lat, 50), launch_to_token_us_p90=pct(lat, 90),
                gpu_us_p50=pct(gpu_us, 50), gpu_us_p90=pct(gpu_us, 90), back_to_back_us_per_step=b2b_us,
                decode_group_us_per_token=r["wall_us"] / max(r["emitted"], 1),
                decode_group_pinned_us_per_token=rp["wall_us"] / max(rp["emitted"], 1),
                decode_pipelined_us_per_token=rq["wall_us"] / max(rq["emitted"], 1),
                decode_group_tokens_agree=bool(toks_gen == toks_pin == toks_pipe))


def bench_lmhead(steps, K=4096, V=102400, rows_list=(1, 4)):
    """LM head (RMSNorm + fp16 GEMV, K x V block-transposed head): us per call
    of plh_logits and plh_greedy, back-to-back on the head's stream, and the
    algorithmic HBM rate (K V 2 head bytes + rows (2 K + V) 4 per call)."""
    from pumice_amd import hip
    from pumice_amd import lmhead as L
    from pumice_amd import sampler as S

    rng = np.random.default_rng(0)
    w = rng.integers(0x2000, 0x3C00, (K // 8, V, 8), dtype=np.uint16) | \
        (rng.integers(0, 2, (K // 8, V, 8), dtype=np.uint16) << 15)
    rmax = max(rows_list)
    x = rng.normal(0, 2, (rmax, K)).astype(np.float32)
    g = rng.normal(1, 0.2, K).astype(np.float32)
    dw, dg, dx = hip.DeviceBuffer.from_array(w), hip.DeviceBuffer.from_array(g), hip.DeviceBuffer.from_array(x)
    del w
    dl = hip.DeviceBuffer(rmax * V * 4)
    head = L.LMHead(dw.ptr, dg.ptr, K, V, rmax)
    s = S.Sampler(V, rmax, stream=head.stream)
    out = {"K": K, "V": V, "head_bytes": K * V * 2}
    try:
        for rows in rows_list:
            nbytes = K * V * 2 + rows * (2 * K + V) * 4
            for name, call in [("logits", lambda: head.logits(dx.ptr, K, rows, dl.ptr, V)),
                               ("greedy", lambda: head.greedy(s, dx.ptr, K, rows, do_increment=0))]:
                for _ in range(3):
                    call()
                e0, e1 = hip.Event(), hip.Event()
                e0.record(head.stream)
                for _ in range(steps):
                    call()
                e1.record(head.stream)
                hip.stream_sync(head.stream)
                us = e0.elapsed_ms(e1) * 1e3 / steps
                out[f"{name}_rows{rows}_us"] = us
                out[f"{name}_rows{rows}_gbps"] = nbytes / (us * 1e-6) / 1e9
        out["logits_rows1_frac"] = out["logits_rows1_gbps"] / HBM_PEAK_GBPS
        # load-time build of this head from a 248,320-row bf16 lm_head pruned
        # to V ids (plh_pack_head: gather + conversions + block transpose)
        src_rows = 248320
        src = hip.DeviceBuffer(src_rows * K * 2)
        try:
            mapping = np.sort(rng.permutation(src_rows)[:V]).astype(np.int32)
            L.pack_head(src.ptr, L.SRC_BF16, src_rows, K, mapping, V, dw.ptr)  # warm
            t0 = time.perf_counter()
            for _ in range(3):
                L.pack_head(src.ptr, L.SRC_BF16, src_rows, K, mapping, V, dw.ptr)
            us = (time.perf_counter() - t0) / 3 * 1e6
            out["pack_head_us"] = us
            out["pack_head_gbps"] = 2 * K * V * 2 / (us * 1e-6) / 1e9
        finally:
            src.free()
    finally:
        s.close()
        head.close()
        for b in (dw, dg, dx, dl):
            b.free()
    return out


def read_ceiling(nbytes, reps=100):
    """The read ceiling: pss_read_ceiling (the resident kernel's access
    pattern -- 1,024-thread workgroups over 400 KiB chunks, 16-byte
    nontemporal loads -- and nothing else) over NBUF rotating buffers of
    `nbytes`, back to back on one stream, bracketed by HIP events."""
    from pumice_amd import hip
    from pumice_amd import sampler as S

    L = S.lib()
    bufs = [hip.DeviceBuffer(nbytes) for _ in range(NBUF)]
    for b in bufs:
        b.fill_u32(0x3F800000)
    nblk = int(L.pss_read_ceiling_blocks(nbytes))
    out = hip.DeviceBuffer(4 * nblk)
    try:
        for i in range(10):
            S._ok(L.pss_read_ceiling(bufs[i % NBUF].ptr, nbytes, out.ptr, None), "pss_read_ceiling")
        hip.synchronize()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(None)
        for i in range(reps):
            S._ok(L.pss_read_ceiling(bufs[i % NBUF].ptr, nbytes, out.ptr, None), "pss_read_ceiling")
        e1.record(None)
        hip.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
    finally:
        out.free()
        for b in bufs:
            b.free()
    return {"bytes": nbytes, "us_per_launch": us, "gbps": nbytes / (us * 1e-6) / 1e9, "workgroups": nblk,
            "how": "pss_read_ceiling, %d rotating buffers, %d launches back to back, HIP events" % (NBUF, reps)}


def _oracle_cflags():
    try:
        txt = open(os.path.join(ROOT, "oracle", "Makefile")).read()
        line = txt.split("CFLAGS =", 1)[1].split("\n", 1)[0]
        cont = txt.split("CFLAGS =", 1)[1].split("\n", 2)[1] if line.rstrip().endswith("\\") else ""
        return "gcc " + " ".join((line.rstrip(" \\") + " " + cont).split())
    except (OSError, IndexError):
        return "unknown"


def cpu_baseline(w, seconds):
    """The reference's CPU path on the box's host cores over a bounded sample
    of the headline rows: O1 (the scalar C restatement of the contract, a full
    sort per row like the reference's sampler_ref) with one thread pinned to
    each CPU this process may run on (capped at 16, the host share of one GPU
    on these boxes), the same on one thread, and O3 (the restated sampler_ref
    itself, src/validation.c:4974-5092, fp64) on all threads."""
    import oracle as O

    allowed = sorted(os.sched_getaffinity(0))
    cpus = allowed[:16]

    def run(kind, cp, budget):
        done, t0 = 0, time.perf_counter()
        while True:
            hist = w.history.copy()
            pos = np.zeros(w.rows, np.uint32)
            rng = w.seeds.copy()
            step = np.zeros(w.rows, np.uint32)
            O.batch_pinned(kind, w.logits, w.params, hist, pos, rng, step, cp)
            done += w.rows
            el = time.perf_counter() - t0
            if el >= budget:
                return done / el, done

    rpsn, nn = run("o1", cpus, seconds)
    rps1, n1 = run("o1", cpus[:1], seconds / 2)
    rps3, n3 = run("o3", cpus, seconds / 2)
    return dict(value=rpsn, unit="rows/s", cores=len(cpus), kind="port",
                sample=f"{nn} headline rows (256 x 102,400 fp32, the headline params) in >= {seconds:.0f} s, "
                       f"{len(cpus)} threads pinned one per CPU",
                cpus_online=os.sysconf("SC_NPROCESSORS_ONLN"), cpus_allowed=len(allowed),
                cpu=_cpu_model(), compiler=_oracle_cflags(),
                one_thread=dict(value=rps1, rows=n1),
                o3_sampler_ref=dict(value=rps3, rows=n3, cores=len(cpus), kind="port of src/validation.c:4974-5092"))


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


SECTIONS = ("headline", "c3", "c4", "c5", "b1")


def traffic_from_pmc(fetch_dir, write_dir, out_path):
    """HBM bytes per launch of the sampler kernels, per bench section, from two
    rocprofv3 --pmc runs of `bench.py --no-cpu-baseline --copy-calib`
    (FETCH_SIZE, then WRITE_SIZE; counters in KiB per dispatch).

    With --copy-calib the bench follows each section (headline, c3, c4, c5,
    batch 1) with ten device-to-device copies of one headline batch: those
    copies split the dispatch sequence into sections, and their known traffic
    (that many bytes read and written) scales each counter.  A section's
    launches are the dispatches of its most frequent sampler kernel; its bytes
    per launch are the sum over all its sampler dispatches / launches."""
    import csv
    import glob
    import re
    from pumice_amd import workloads as WL

    nbytes = 256 * 102400 * 4

    def dispatches(d, counter):
        out = []
        for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(fn)):
                if r["Counter_Name"] == counter:
                    out.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
        out.sort()
        return out

    def short(k):
        m = re.search(r"(pss_\w+|plh_\w+)(<[^>]*>)?", k)
        return (m.group(1) + (m.group(2) or "")) if m else k

    def is_calib(k, v):
        return "copyBuffer" in k and v * 1024 > nbytes / 4

    def is_sampler(k):
        s = short(k)
        return s.startswith("pss_") and not s.startswith(("pss_fill_u32", "pss_read_kernel"))

    per = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        seq = dispatches(d, counter)
        copy = [v for _, k, v in seq if is_calib(k, v)]
        if not copy:
            raise SystemExit(f"{d}: no calibration copy dispatch found")
        scale = nbytes / (float(np.mean(copy)) * 1024.0)
        segs, cur = [], []
        for _, k, v in seq:
            if is_calib(k, v):
                if cur:
                    segs.append(cur)
                cur = []
            elif is_sampler(k):
                cur.append((short(k), v))
        if cur:
            segs.append(cur)
        per[counter] = {"copy_kib": float(np.mean(copy)), "scale": scale, "segments": segs}
    nseg = len(per["FETCH_SIZE"]["segments"])
    if nseg != len(per["WRITE_SIZE"]["segments"]) or nseg > len(SECTIONS):
        raise SystemExit("the two runs do not have the same sections")
    gens = {"headline": lambda: WL.headline(seed=0), "c3": lambda: WL.c3(seed=3), "c4": lambda: WL.c4(seed=4),
            "c5": lambda: WL.c5(seed=5), "b1": lambda: WL.c2(seed=2, rows=1, steps=1)[0]}
    sections = {}
    for i in range(nseg):
        name = SECTIONS[i]
        w = gens[name]()
        entry = {"algorithmic_bytes_per_launch": int(w.bytes_per_row() * w.rows)}
        total = 0.0
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            seg = per[counter]["segments"][i]
            counts = {}
            for k, v in seg:
                counts[k] = counts.get(k, 0) + 1
            launches = max(counts.values())
            kib = sum(v for _, v in seg) / launches
            entry[counter] = {"kib_per_launch": kib, "launches": launches}
            entry["kernels"] = sorted(counts)
            total += kib * 1024.0 * per[counter]["scale"]
        entry["hbm_bytes_per_launch"] = total
        entry["ratio"] = total / entry["algorithmic_bytes_per_launch"]
        sections[name] = entry
    head = sections["headline"]
    res = {"kernel": head["kernels"][0].split("<")[0], "workload": "headline 256 x 102,400 fp32",
           "calibration_copy_bytes": nbytes,
           "scale": {c: per[c]["scale"] for c in per}, "copy_kib": {c: per[c]["copy_kib"] for c in per},
           "sections": sections, "row_kernel_hbm_bytes_per_launch": head["hbm_bytes_per_launch"]}
    md = [
        "# HBM traffic of the sampler kernels, per bench configuration",
        "",
        "Commands (from the repository root on the MI355X box; then, on any host,",
        "`python3 bench.py --traffic-from <fetch dir> <write dir>` wrote this file):",
        "",
        "    cd /tmp && export TMPDIR=/tmp",
        "    timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE -d $REPO/gpurun_out/prof_fetch -o run --output-format csv \\",
        "        -- python3 $REPO/bench.py --no-cpu-baseline --steps 10 --warmup 2 --latency-steps 20 --copy-calib",
        "    timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE -d $REPO/gpurun_out/prof_write -o run --output-format csv \\",
        "        -- python3 $REPO/bench.py --no-cpu-baseline --steps 10 --warmup 2 --latency-steps 20 --copy-calib",
        "",
        "Calibration: a device-to-device copy of one headline batch (%d bytes read and written) reads"
        % nbytes,
        "FETCH_SIZE %.1f KiB and WRITE_SIZE %.1f KiB per dispatch, so the counters are scaled by %.4f and %.4f."
        % (per["FETCH_SIZE"]["copy_kib"], per["WRITE_SIZE"]["copy_kib"], per["FETCH_SIZE"]["scale"],
           per["WRITE_SIZE"]["scale"]),
        "Algorithmic bytes per launch: rows x (V x element size + 4 x window + 44).",
        "",
        "| config | kernels | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes per launch (scaled) | algorithmic | ratio |",
        "|---|---|---|---|---|---|---|",
    ]
    for name, e in sections.items():
        md.append("| %s | %s | %.1f | %.1f | %.0f | %d | %.3f |" % (
            name, ", ".join("`%s`" % k for k in e["kernels"]), e["FETCH_SIZE"]["kib_per_launch"],
            e["WRITE_SIZE"]["kib_per_launch"], e["hbm_bytes_per_launch"], e["algorithmic_bytes_per_launch"],
            e["ratio"]))
    md += ["", "```json", json.dumps(res, indent=1), "```", ""]
    with open(out_path, "w") as f:
        f.write("\n".join(md))
    print(json.dumps(res))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # an idle GPU runs the first few ms of launches about 5% slower while its
    # clocks rise; 2,000 untimed launches (about 50 ms of the headline) reach
    # the steady rate (200 timed launches: 25.0-25.6 us after 20 warmups,
    # 23.8-24.0 us after 2,000, on one box)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--latency-steps", type=int, default=1000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline only (c3/c4/c5 and latency skipped)")
    ap.add_argument("--latency-only", action="store_true",
                    help="only the batch-1 latency section (for kernel traces of the small-batch form)")
    ap.add_argument("--lmhead-only", action="store_true",
                    help="only the LM-head section (for kernel traces of plh_gemv_kernel)")
    ap.add_argument("--lmhead-steps", type=int, default=50)
    ap.add_argument("--general", action="store_true", help="force the general kernel")
    ap.add_argument("--split", action="store_true", help="force the two-kernel form")
    ap.add_argument("--fused", action="store_true", help="force the LDS-staged fused form")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run device-to-device copies of one headline batch (traffic calibration)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU: turn two rocprofv3 --pmc output directories into "
                         "profiles/sampler_traffic_by_config.md and exit")
    args = ap.parse_args()
    if args.traffic_from:
        traffic_from_pmc(args.traffic_from[0], args.traffic_from[1], os.path.join(ROOT, "profiles", TRAFFIC_MD))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(rows shard with no exchange; see the sharding design). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    from pumice_amd import sampler as S
    from pumice_amd import workloads as WL

    if args.lmhead_only:
        log("lm head (K 4096 x V 102400)")
        print(json.dumps({"lmhead": bench_lmhead(args.lmhead_steps)}), flush=True)
        if args.copy_calib:
            copy_calibration(256 * 102400 * 4)
            log("copy calibration:", 256 * 102400 * 4, "bytes per copy")
        return
    if args.latency_only:
        log("latency (batch 1)")
        lat = bench_latency(args.latency_steps)
        print(json.dumps({"latency_b1": lat}), flush=True)
        return
    flags = (S.ENQ_GENERAL if args.general else S.ENQ_SPLIT if args.split else
             S.ENQ_FUSED if args.fused else 0)
    kernel = ("general" if args.general else "split" if args.split else "fused" if args.fused
              else "resident")
    log("generating headline workload")
    head = WL.headline(seed=0)
    log("headline: 256 x 102400 fp32")
    h = bench_batched(head, args.steps, args.warmup, flags)
    log("headline", json.dumps(h))
    if args.copy_calib:
        copy_calibration(head.logits.nbytes)
        log("copy calibration:", head.logits.nbytes, "bytes per copy")
    extra = {}
    if not args.no_extra:
        for name, gen in [("c3", lambda: WL.c3(seed=3)), ("c4", lambda: WL.c4(seed=4)),
                          ("c5", lambda: WL.c5(seed=5))]:
            log("workload", name)
            extra[name] = bench_batched(gen(), max(args.steps // 2, 10), args.warmup, flags)
            log(name, json.dumps(extra[name]))
            if args.copy_calib:
                copy_calibration(head.logits.nbytes)
        log("latency (batch 1)")
        extra["latency_b1"] = bench_latency(args.latency_steps)
        log("latency", json.dumps(extra["latency_b1"]))
        if args.copy_calib:
            copy_calibration(head.logits.nbytes)
        log("lm head (K 4096 x V 102400)")
        extra["lmhead"] = bench_lmhead(args.lmhead_steps)
        log("lmhead", json.dumps(extra["lmhead"]))
    log("read ceiling")
    ceiling = read_ceiling(head.logits.nbytes)
    log("read ceiling", json.dumps(ceiling))
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(head, args.cpu_seconds)
        log("cpu", json.dumps(cpu))

    traffic = None
    traffic_by = {}
    tpath = os.path.join(ROOT, "profiles", TRAFFIC_MD)
    if os.path.exists(tpath):
        with open(tpath) as f:
            txt = f.read()
        if "```json" in txt:
            tj = json.loads(txt.split("```json", 1)[1].split("```", 1)[0])
            # counters read for the kernel form this run times, else none
            kname = {"resident": "pss_res_kernel", "fused": "pss_row_kernel"}.get(kernel)
            if tj.get("kernel") == kname:
                traffic = tj.get("row_kernel_hbm_bytes_per_launch")
                traffic_by = {n: e["hbm_bytes_per_launch"] for n, e in tj.get("sections", {}).items()}
    # dominant (fused: only) kernel: algorithmic bytes per launch / mean
    # per-launch time from HIP events on the sampler's stream bracketing the
    # timed back-to-back launches (events around single launches, which add
    # the dispatch, are in headline.launch_ms_*)
    achieved = h["stream_gbps"]
    line = {
        "metric": "sampled rows/sec + HBM GB/s at V=102,400 (B=256); p50 µs/token at B=1",
        "value": h["rows_per_s"],
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy: N(0,3^2) logits, uniform 64-id windows); no dataset",
        "config": {
            "workload": "headline: 256 rows x V=102,400 fp32 logits, rep 1.1 + presence 0.5 over a "
                        "64-id window, T 0.8, top-k 40, top-p 0.95, min-p 0.05, xorshift32 seeds 0..255",
            "rows": 256, "vocab": 102400, "kernel": kernel, "kernel_b1": "small",
        },
        "hbm_gbps": h["wall_gbps"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic},
        "read_ceiling_gbps": ceiling["gbps"],
        "read_ceiling": ceiling,
        "roofline_by_config": {
            name: {"achieved": extra[name]["stream_gbps"], "frac": extra[name]["stream_gbps"] / HBM_PEAK_GBPS,
                   "us_per_launch": extra[name]["stream_ms_per_launch"] * 1e3,
                   "traffic": traffic_by.get(name)}
            for name in ("c3", "c4", "c5") if name in extra},
        "cpu_baseline": cpu,
        "p50_us_per_token_b1": extra.get("latency_b1", {}).get("launch_to_token_us_p50"),
        "headline": h,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
