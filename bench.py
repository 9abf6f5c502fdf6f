"""Benchmark of the SJ-KVaRN codec hot path on one MI355X (BASELINE.json metric).

  step (the timed unit, `value`): one adaptive-tail commit of configs[1]: 4096 tokens (32 groups x 4 KV
      heads = 128 records) sealed at 4/4 scalar, D = 256, straight out of the tq6_0 staging ring in HBM
      (sjk_hip_commit). value = sealed tokens/s = 4096 / commit time.
  attention: decode width 4, 16 query heads on 4 KV heads, D = 256, N = 100,000 reached by
      the default decode schedule (B = 94,336, tail 5,664, fp16 sink 128). Reported in us and HBM GB/s;
      `roofline` is this kernel's: algorithmic bytes per call / measured time / 8 TB/s. The 113 MB cache
      fits the 256 MB Infinity Cache, so timed calls rotate over 8 copies of the cache (0.9 GB).
  attention_3_3t / attention_3_3s / attention_d128: the same schedule with the 3/3 trellis body, the 3/3 scalar
      body, and the 4/4 body at head dimension 128 (8 KV heads, 32 query heads, width 4), timed the same way (not
      the roofline line). attention_scalar_bodies (on request, --attn-bodies 2/4s,4/2sd128,...): the other scalar
      bodies, the same way.
  append: tq6_0 append of 4 positions x 4 heads (K and V) with the Hadamard fused.
  cpu_baseline: the reference's own C code (sj_kvarn.h compiled as-is into oracle/_ref/libsjk_ref.so,
      -O2, in the build container; kind "reference") or, where that library is absent, the oracle (the
      C99 restatement, kind "port"): layer_seal on the same ring bytes, single-thread and on 16 threads
      (the box's CPU share for one GPU) with records split over threads, and layer_attend_row for all 64
      (query row, head) pairs on a copy of the same 100K cache. Median and spread of 5 runs each, with the
      CPU model, the compiler and the flags.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-attn] [--no-seal] [--no-pool]
       [--no-host-seal] [--attn-bodies 4/4,3/3t,4/4d128,3/3s]
"""
import argparse
import ctypes as C
import json
import os
import re
import subprocess
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sj-kvarn-codec_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import sjk  # noqa: E402
import inputs  # noqa: E402
import contexts  # noqa: E402

METRIC = "sealed tokens/s per 4096-tok commit; 100K-ctx decode attn µs + HBM GB/s"
HBM_PEAK_GBS = 8000.0
D, H, S, G = 256, 4, 128, 128
TAIL, TAIL_MAX = 4096, 8192


def log(*a):
    print(*a, file=sys.stderr, flush=True)


make_layer, store, decode_schedule_B = contexts.make_layer, contexts.store, contexts.decode_schedule_B


def timed(dev, stream, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    dev.hip.hipStreamSynchronize(stream)
    e0, e1 = dev.event(), dev.event()
    t0 = time.perf_counter()
    dev.hip.hipEventRecord(e0, stream)
    for _ in range(steps):
        fn()
    dev.hip.hipEventRecord(e1, stream)
    ms = dev.elapsed_ms(e0, e1) / steps
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return ms, wall


# ------------------------------------------------------------------------------------------------
# CPU baseline (oracle) helpers
# ------------------------------------------------------------------------------------------------

def oracle_layer_from_device(orc, cabi, dev, cfg, L, B_body_groups):
    return contexts.oracle_layer_from_device(orc, dev, cfg, L, B_body_groups)


CPU_RUNS = 5


def cpu_threads():
    """Threads of the all-cores figures: the host CPUs this process may use, at most 16 (the CPU share of one
    GPU on the benchmark boxes, whatever the host's own count)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def cpu_info(kind):
    """CPU model, host CPU count, the compiler of the CPU libraries and their flags (oracle/Makefile)."""
    info = {"cpu_model": None, "host_cpus": os.cpu_count(), "compiler": None, "flags": None}
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["cpu_model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        info["compiler"] = subprocess.run(["gcc", "--version"], capture_output=True, text=True,
                                          timeout=10).stdout.splitlines()[0]
    except (OSError, IndexError, subprocess.SubprocessError):
        pass
    try:
        want = "REFFLAGS" if kind == "reference" else "CFLAGS"
        for line in open(os.path.join(ROOT, "oracle", "Makefile")):
            if line.split("=")[0].strip() == want:
                info["flags"] = line.split("=", 1)[1].strip()
    except OSError:
        pass
    return info


def spread(ts):
    """median, min and max of a list of run times (s)"""
    ts = sorted(ts)
    return float(np.median(ts)), ts[0], ts[-1]


def cpu_lib(cabi):
    """(library, kind): the reference compiled from its own header where it was built, else the oracle"""
    ref = cabi.reference()
    return (ref, "reference") if ref is not None else (cabi.oracle(), "port")


def cpu_seal_runs(lib, cabi, dev, cfg, L, n_threads, n_groups, runs):
    """layer_seal over n_groups groups (x4 heads), split over n_threads threads with one layer per thread,
    `runs` times (the same ring bytes give the same records): (wall seconds of each run, layers)."""
    layers = [oracle_layer_from_device(lib, cabi, dev, cfg, L, 0) for _ in range(n_threads)]
    per = [list(range(n_groups))[i::n_threads] for i in range(n_threads)]

    def work(i):
        for g in per[i]:
            lib.layer_seal(C.byref(layers[i]), S + g * G, S + (g + 1) * G)

    ts = []
    for _ in range(runs):
        ths = [threading.Thread(target=work, args=(i,)) for i in range(n_threads)]
        t0 = time.perf_counter()
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        ts.append(time.perf_counter() - t0)
    return ts, layers


def config1_round_trip(lib, dev, orc, cabi):
    """one 128-token group (1 KV head, D = 128, 4/4, K outlier channels 3 and 77 x12) sealed on the
    device and decoded with sjk_hip_decode: the record and the decoded rows against the oracle's, and the round-trip
    MSE of K and V against the fp16 rows sealed (absolute, and over the rows' mean square)."""
    K, V = inputs.kv_rows_c1(seed=0)
    Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
    lay = sjk.Layout()
    sjk.check(lib.sj_kvarn_layout_init(C.byref(lay), 128, 128, 4, 4, 0), "layout_init")
    dK, dV, dR = dev.put(Kh), dev.put(Vh), dev.alloc(lay.bytes)
    sjk.check(lib.sjk_hip_seal(C.byref(lay), dK, dV, 128, 1, 1, 16, dR, None), "sjk_hip_seal")
    dk, dv = dev.alloc(128 * 128 * 4), dev.alloc(128 * 128 * 4)
    sjk.check(lib.sjk_hip_decode(C.byref(lay), dR, 1, dk, dv, None), "sjk_hip_decode")
    dev.sync()
    rec = dev.get(dR, lay.bytes, np.uint8)
    gk = dev.get(dk, 128 * 128 * 4, np.float32).reshape(128, 128)
    gv = dev.get(dv, 128 * 128 * 4, np.float32).reshape(128, 128)
    olay = orc.layout(128, 128, 4, 4, 0)
    want = np.zeros(olay.bytes, np.uint8)
    work = np.zeros(orc.seal_workspace_bytes(C.byref(olay)), np.uint8)
    orc.seal_group(C.byref(olay), cabi.ptr(Kh, cabi.u16p), cabi.ptr(Vh, cabi.u16p), 128, 16, cabi.ptr(want),
                   work.ctypes.data_as(C.c_void_p))
    ok, ov = np.zeros((128, 128), np.float32), np.zeros((128, 128), np.float32)
    for t in range(128):
        orc.decode_k_row(C.byref(olay), cabi.ptr(want), t, cabi.ptr(ok[t], cabi.f32p))
        orc.decode_v_row(C.byref(olay), cabi.ptr(want), t, cabi.ptr(ov[t], cabi.f32p))
    mk, rk = inputs.round_trip_mse(Kh, gk)
    mv, rv = inputs.round_trip_mse(Vh, gv)
    for d in (dK, dV, dR, dk, dv):
        dev.free(d)
    return {"workload": "configs[0]: seal then decode one 128-token group, 1 KV head, D=128, 4/4 scalar body, K "
                        "channels 3 and 77 x12 (seed 0)", "record_bytes": int(lay.bytes),
            "record_equal_oracle": bool(np.array_equal(rec, want)),
            "decoded_rows_equal_oracle": bool(np.array_equal(gk.view(np.uint32), ok.view(np.uint32)) and
                                              np.array_equal(gv.view(np.uint32), ov.view(np.uint32))),
            "round_trip_mse_k": round(mk, 6), "round_trip_mse_v": round(mv, 6),
            "round_trip_rel_mse_k": round(rk, 6), "round_trip_rel_mse_v": round(rv, 6)}


def records_equal(dev, L, layers, n_groups):
    """records of the device layer L equal to those the CPU layers sealed (groups split round-robin over them)"""
    nb = L.lay.bytes
    got = dev.get(C.c_void_p(L.body), n_groups * H * nb, np.uint8)
    want = np.zeros_like(got)
    for i in range(len(layers)):
        base = C.cast(layers[i].body, C.c_void_p).value
        for g in range(i, n_groups, len(layers)):
            off = g * H * nb
            C.memmove(want[off:].ctypes.data, C.c_void_p(base + off), H * nb)
    return int(sum(np.array_equal(got[r * nb:(r + 1) * nb], want[r * nb:(r + 1) * nb]) for r in range(n_groups * H)))


def host_buffer_seal(lib, dev, stream, lay, K, V, dk, dv, dbody, reps=5):
    """The fp16-rows seal when the caller hands over host memory (not the resident rate that `value` is):
    (1) sjk_hip_seal with the commit's rows copied in and the records copied out (pageable buffers,
    synchronous hipMemcpy), wall clock; (2) the drop-in host call sj_kvarn_seal_group once per record
    (each call allocates its device buffers and copies synchronously), wall clock. Both must give the
    bytes of the resident seal."""
    n_tok, H, D = K.shape
    G, n_rec = 128, (K.shape[0] // 128) * H
    kh = np.ascontiguousarray(K.astype(np.float16))
    vh = np.ascontiguousarray(V.astype(np.float16))
    rec = np.empty(n_rec * lay.bytes, np.uint8)
    ref = dev.get(dbody, rec.nbytes, np.uint8)

    def pcie():
        t0 = time.perf_counter()
        dev.upload(dk, kh)
        dev.upload(dv, vh)
        sjk.check(lib.sjk_hip_seal(C.byref(lay), dk, dv, H * D, H, n_tok // G, 16, dbody, stream), "sjk_hip_seal")
        dev.hip.hipStreamSynchronize(stream)
        dev._ck(dev.hip.hipMemcpy(rec.ctypes.data, dbody, rec.nbytes, dev.D2H), "hipMemcpy D2H")
        return time.perf_counter() - t0
    pcie()
    t_pcie = sorted(pcie() for _ in range(reps))[reps // 2]
    eq_pcie = bool(np.array_equal(rec, ref))

    u16p, u8p = C.POINTER(C.c_uint16), C.POINTER(C.c_uint8)

    def per_record():
        t0 = time.perf_counter()
        for g in range(n_tok // G):
            for h in range(H):
                off = (g * G * H + h) * D * 2                     # bytes to row g*G, head h
                r = g * H + h
                lib.sj_kvarn_seal_group(C.byref(lay), C.cast(kh.ctypes.data + off, u16p),
                                        C.cast(vh.ctypes.data + off, u16p), H * D, 16,
                                        C.cast(rec.ctypes.data + r * lay.bytes, u8p), None)
        return time.perf_counter() - t0
    rec[:] = 0
    per_record()
    t_rec = sorted(per_record() for _ in range(3))[1]
    eq_rec = bool(np.array_equal(rec, ref))
    h2d, d2h = kh.nbytes + vh.nbytes, rec.nbytes
    return {"pcie_inclusive": {"ms_per_4096_tokens": round(t_pcie * 1e3, 3),
                               "tokens_per_s": round(n_tok / t_pcie, 1), "h2d_bytes": h2d, "d2h_bytes": d2h,
                               "records_equal_resident": eq_pcie,
                               "workload": "host fp16 rows -> hipMemcpy -> sjk_hip_seal -> hipMemcpy -> host records "
                                           "(pageable), median of %d, wall clock" % reps},
            "seal_group_per_record": {"ms_per_4096_tokens": round(t_rec * 1e3, 2),
                                      "ms_per_record": round(t_rec * 1e3 / n_rec, 3),
                                      "records_equal_resident": eq_rec,
                                      "workload": "%d calls of the drop-in sj_kvarn_seal_group (host arrays), median "
                                                  "of 3, wall clock" % n_rec}}


def measured_traffic():
    """HBM bytes per attention call measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (profiles/, calibrated on a
    copy kernel); None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "attention_traffic_pmc.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


N_COPIES = 8


def attention_context(lib, dev, stream, N, B, commits, bk, bv, body, d=D, h=H, n_head=16):
    """The configs[3] decode-schedule context of N positions (tests/contexts.py; head dimension d, h KV heads),
    plus N_COPIES - 1 device copies of its sink, ring and body, so that timed calls rotate over N_COPIES x 113 MB
    (0.9 GB) and stream from HBM rather than the 256 MB Infinity Cache."""
    cfg, Lc, v0, B2, n_body, tail, alg_bytes = contexts.attention_context(lib, dev, stream, N, bk, bv, body, log=log,
                                                                          d=d, h=h, n_head=n_head)
    assert B2 == B
    copies, extra = [v0], []
    for _ in range(N_COPIES - 1):
        v = sjk.View.from_buffer_copy(bytes(v0))
        for name, nb in (("sink", S * h * d * 4), ("ring", Lc.cap * h * 2 * Lc.stage_bytes),
                         ("body", n_body * h * Lc.lay.bytes)):
            p = dev.alloc(nb, zero=False)
            dev.hip.hipMemcpy(p, C.c_void_p(getattr(v0, name)), nb, 3)
            setattr(v, name, p.value)
            extra.append(p)
        copies.append(v)
    return cfg, Lc, v0, n_body, tail, alg_bytes, (copies, extra)


def free_context(lib, dev, ctx):
    for p in ctx[6][1]:
        dev.free(p)
    lib.sj_kvarn_layer_free(C.byref(ctx[1]))


def time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args):
    views = copies[0]
    it = [0]

    def attend():
        v = views[it[0] % len(views)]
        it[0] += 1
        return lib.sjk_hip_attend(C.byref(v), B, N, qpos0, n_q, n_head, dq, 1.0 / 16.0, do, stream)

    sjk.check(attend(), "attend")
    steps_a = args.attn_calls or max(50, args.steps) * len(views)
    # a decode loop calls attention back to back: 2000 untimed calls (~70 ms) bring the clocks to that state
    # (after 200 the calls were still ~10% slower than after 400 more)
    log("[bench] attention: timing %d calls after %d untimed ones" % (steps_a, args.attn_warmup))
    ms, _ = timed(dev, stream, attend, steps_a, args.attn_warmup)
    # leave the output of copy 0 (the cache the oracle is given) in `do`
    sjk.check(lib.sjk_hip_attend(C.byref(views[0]), B, N, qpos0, n_q, n_head, dq, 1.0 / 16.0, do, stream), "attend")
    dev.hip.hipStreamSynchronize(stream)
    return ms


def oracle_attend(orc, cabi, OL, q, B, N, qpos0, pairs, n_thr, gq=4):
    """oracle layer_attend_row for (row, head) pairs on n_thr threads (GQA gq:1): (outputs, wall seconds)"""
    want = {}

    def att(pair):
        iq, hq = pair
        o = np.zeros(q.shape[2], np.float32)
        qq = np.ascontiguousarray(q[iq, hq])
        orc.layer_attend_row(C.byref(OL), B, N, cabi.ptr(qq, cabi.f32p), hq // gq, qpos0 + iq, 1.0 / 16.0,
                             cabi.ptr(o, cabi.f32p))
        want[pair] = o

    ths = [threading.Thread(target=lambda k=k: [att(p) for p in pairs[k::n_thr]]) for k in range(n_thr)]
    t0 = time.perf_counter()
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    return want, time.perf_counter() - t0


def time_shapes(lib, dev, stream, copies, B, N, d, h, ctx_bytes, gbs16, shapes, args):
    """Other query shapes on the same context: for each (name, n_q, n_head) the call time, its algorithmic bytes
    (the context once, Q fp16 and O fp32 of the shape) over that time, and that rate against the 16-row call's.
    Returns (report, {name: (q, output, qpos0)}) for the parity check."""
    rep, outs = {}, {}
    for name, sq, sh in shapes:
        rows = sq * sh // h
        qs = np.random.default_rng(40 + sq + sh).standard_normal((sq, sh, d)).astype(np.float32)
        dqs, dos = dev.put(qs), dev.alloc(qs.nbytes)
        ms = time_attention(lib, dev, stream, copies, B, N, N - sq, dqs, dos, sq, sh, args)
        nb = ctx_bytes + sq * sh * d * (2 + 4)
        gbs = nb / (ms * 1e-3) / 1e9
        rep[name] = {"n_q": sq, "n_head": sh, "rows_per_kv_head": rows, "us_per_call": round(ms * 1e3, 2),
                     "algorithmic_bytes": int(nb), "hbm_GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "GBps_vs_16_row_call": round(gbs / gbs16, 3),
                     "path": ("one 16-row job" if rows <= 16 else
                              "%d 16-row jobs side by side in one launch, each reading the context (the bytes count it "
                              "once)" % ((rows + 15) // 16))}
        outs[name] = (qs, dev.get(dos, qs.nbytes, np.float32).reshape(qs.shape), N - sq)
        dev.free(dqs)
        dev.free(dos)
    return rep, outs


def shapes_parity(orc, cabi, OL, B, N, h, outs):
    """max |gpu - oracle| / (1e-3 + 1e-3 |oracle|) over the first and last rows of every shape"""
    worst = 0.0
    for name, (qs, got, qpos0) in outs.items():
        sq, sh = qs.shape[0], qs.shape[1]
        pairs = sorted({(0, 0), (0, sh - 1), (sq - 1, 0), (sq - 1, sh - 1), (sq // 2, sh // 2)})
        want, _ = oracle_attend(orc, cabi, OL, qs, B, N, qpos0, pairs, len(pairs), gq=sh // h)
        worst = max(worst, max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs))
    return round(worst, 4)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-attn", action="store_true")
    ap.add_argument("--no-seal", action="store_true")
    ap.add_argument("--no-pool", action="store_true")
    ap.add_argument("--no-host-seal", action="store_true", help="skip the seal from host buffers (PCIe-inclusive rates)")
    ap.add_argument("--pool-steps", type=int, default=2048, help="decode rounds of the configs[4] pool stress")
    ap.add_argument("--attn-bodies", default="4/4,3/3t,4/4d128,3/3s",
                    help="attention bodies to time at 100K (4/4, 3/3t, 4/4d128: the 4/4 body at D = 128, 8 KV heads, "
                         "3/3s: the 3/3 scalar body; also 3/3td128: the 3/3 trellis body at D = 128, 8 KV heads, and "
                         "the other scalar bodies, e.g. 2/4s or 4/2sd128)")
    ap.add_argument("--attn-warmup", type=int, default=2000, help="untimed attention calls before the timed ones")
    ap.add_argument("--attn-calls", type=int, default=0, help="timed attention calls (0: 50 per cache copy)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="also run 4 device-to-device copies of MIB MiB (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box in this build has one MI355X and the codec path has no "
              "multi-GPU leg. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    lib = sjk.load()
    dev = sjk.Device()
    stream = dev.stream()
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "scaling": "weak", "dtype": "f32", "data": "synthetic (seeded N(0,1) K/V, 2% K outlier channels x10, "
           "lognormal(0,0.3) K token norms)"}

    import cabi
    orc = cabi.oracle()
    L = L3 = None
    if not args.no_seal:
        out["config1"] = config1_round_trip(lib, dev, orc, cabi)
        # ---------------- C2: 4096-token 4/4 commit out of the ring ----------------
        log("[bench] C2: building the staging ring (8320 positions, fused rotation + tq6_0 append)")
        cfg, L = make_layer(lib, n_ctx=16384, n_ubatch=512)
        view = lib.sjk_layer_view(C.byref(L))
        n_pos = S + TAIL_MAX
        K, V = inputs.kv_rows(n_pos, H, D, seed=2024)
        store(lib, dev, view, K, V, 0, stream)
        B_from, B_to = S, S + 4096
        commit = lambda: lib.sjk_hip_commit(C.byref(view), 1, B_from, B_to, 16, stream)  # noqa: E731
        sjk.check(commit(), "sjk_hip_commit")
        dev.hip.hipStreamSynchronize(stream)
        log("[bench] C2: timing %d commits (warmup %d)" % (args.steps, args.warmup))
        ms, wall = timed(dev, stream, commit, args.steps, args.warmup)
        out["value"] = round(4096.0 / (ms * 1e-3), 1)
        out["unit"] = "tokens/s"
        out["ms_per_step"] = round(ms, 4)
        out["wall_ms_per_step"] = round(wall, 4)
        out["config"] = {"workload": "configs[1]: single-layer 4096-token seal commit out of the tq6_0 ring, 4/4 scalar "
                         "body, 4 KV heads, D=256, G=128, 16 balance iterations (128 records)",
                         "records": 128, "record_bytes": int(L.lay.bytes), "target_ms": 10.0}
        # the reference's published numbers for this exact commit (its README.md:55-57; RTX 3090 Ti)
        out["vs_baseline"] = round(out["value"] / (4096.0 / 0.953), 2)
        out["vs_baseline_ref"] = "reference CUDA kernels, 953 ms per commit on RTX 3090 Ti (README.md:55-57)"
        out["vs_fork_tuned"] = round(out["value"] / (4096.0 / 0.0104), 2)

        # the fp16-rows -> records core (sjk_hip_seal, the sj_kvarn_cuda_seal contract) on the same rows
        dkf = dev.put(K[S:S + 4096].astype(np.float16))         # [4096][H][D]
        dvf = dev.put(V[S:S + 4096].astype(np.float16))
        dbody = dev.alloc(128 * L.lay.bytes, zero=False)
        seal = lambda: lib.sjk_hip_seal(C.byref(L.lay), dkf, dvf, H * D, H, 32, 16, dbody, stream)  # noqa: E731
        sjk.check(seal(), "sjk_hip_seal")
        ms_s, _ = timed(dev, stream, seal, args.steps, args.warmup)
        out["seal_fp16_rows"] = {"ms_per_4096_tokens": round(ms_s, 4), "tokens_per_s": round(4096.0 / (ms_s * 1e-3), 1),
                                 "workload": "sjk_hip_seal of 4096 fp16 rows x 4 heads (128 records), no ring"}
        if not args.no_host_seal:
            out["seal_host_buffers"] = host_buffer_seal(lib, dev, stream, L.lay, K[S:S + 4096], V[S:S + 4096], dkf, dvf,
                                                        dbody)

        # 3/2 trellis commit on the same ring bytes
        cfg3, L3 = make_layer(lib, n_ctx=16384, n_ubatch=512, bk=3, bv=2, body=1)
        view3 = lib.sjk_layer_view(C.byref(L3))
        store(lib, dev, view3, K, V, 0, stream)
        commit3 = lambda: lib.sjk_hip_commit(C.byref(view3), 1, B_from, B_to, 16, stream)  # noqa: E731
        sjk.check(commit3(), "sjk_hip_commit 3/2t")
        log("[bench] C3: timing 3/2 trellis commits")
        ms3, _ = timed(dev, stream, commit3, max(3, args.steps // 2), 1)
        out["trellis_3_2"] = {"ms_per_commit": round(ms3, 4), "tokens_per_s": round(4096.0 / (ms3 * 1e-3), 1),
                              "workload": "configs[2]: same commit, 3/2 trellis body", "fork_tuned_ms": 16.9,
                              "reference_cuda_ms": 3399}

        # CPU baseline on the same ring bytes, and parity of the whole timed commit against it
        if not args.no_cpu:
            clib, kind = cpu_lib(cabi)
            n_threads = cpu_threads()
            n_groups, st_groups = 32, 8
            log("[bench] CPU baseline (%s): layer_seal of the commit's %d groups on %d threads, %d runs" %
                (kind, n_groups, n_threads, CPU_RUNS))
            ts, layers = cpu_seal_runs(clib, cabi, dev, cfg, L, n_threads, n_groups, CPU_RUNS)
            out["parity_records_checked"] = int(n_groups * H)
            out["parity_records_equal"] = records_equal(dev, L, layers, n_groups)
            for ly in layers:
                clib.layer_free(C.byref(ly))
            log("[bench] CPU baseline (%s): layer_seal of %d groups on one thread, %d runs" %
                (kind, st_groups, CPU_RUNS))
            ts1, layers = cpu_seal_runs(clib, cabi, dev, cfg, L, 1, st_groups, CPU_RUNS)
            for ly in layers:
                clib.layer_free(C.byref(ly))
            med, lo, hi = spread(ts)
            med1, lo1, hi1 = spread(ts1)
            tok = n_groups * G
            out["cpu_baseline"] = {
                "value": round(tok / med, 1), "unit": "tokens/s", "cores": n_threads, "kind": kind,
                "sample": "the whole commit (32 groups x 4 heads = 128 records) sealed by layer_seal from the same ring "
                          "bytes, groups split over %d threads; median of %d runs (%.3f s, spread %.3f-%.3f s)" %
                          (n_threads, CPU_RUNS, med, lo, hi),
                "runs": CPU_RUNS, "spread_tokens_per_s": [round(tok / hi, 1), round(tok / lo, 1)],
                "single_thread": {"value": round(st_groups * G / med1, 1), "unit": "tokens/s",
                                  "ms_per_commit": round(med1 * n_groups / st_groups * 1e3, 1),
                                  "sample": "%d groups (%d records) on one thread, median of %d runs (%.3f s, spread "
                                            "%.3f-%.3f s), scaled to the 32-group commit" %
                                            (st_groups, st_groups * H, CPU_RUNS, med1, lo1, hi1),
                                  "spread_tokens_per_s": [round(st_groups * G / hi1, 1), round(st_groups * G / lo1, 1)]}}
            out["cpu_baseline"].update(cpu_info(kind))
            if kind == "reference":
                # the port (the oracle the tests check against) on the same single-thread sample
                tsp, layers = cpu_seal_runs(orc, cabi, dev, cfg, L, 1, st_groups, 3)
                for ly in layers:
                    orc.layer_free(C.byref(ly))
                out["cpu_baseline"]["single_thread"]["port_over_reference_time"] = round(spread(tsp)[0] / med1, 3)
            # the 3/2 trellis commit from the same ring bytes (its Viterbi makes a CPU record ~4x the
            # 4/4's time: the whole commit on all threads, 2 groups on one thread)
            n3, st3 = 32, 2
            log("[bench] CPU baseline (%s): 3/2 trellis layer_seal of %d groups on %d threads, %d runs" %
                (kind, n3, n_threads, CPU_RUNS))
            ts3, layers = cpu_seal_runs(clib, cabi, dev, cfg3, L3, n_threads, n3, CPU_RUNS)
            eq3 = records_equal(dev, L3, layers, n3)
            for ly in layers:
                clib.layer_free(C.byref(ly))
            log("[bench] CPU baseline (%s): 3/2 trellis layer_seal of %d groups on one thread, %d runs" %
                (kind, st3, CPU_RUNS))
            ts31, layers = cpu_seal_runs(clib, cabi, dev, cfg3, L3, 1, st3, CPU_RUNS)
            for ly in layers:
                clib.layer_free(C.byref(ly))
            med, lo, hi = spread(ts3)
            med1, lo1, hi1 = spread(ts31)
            out["trellis_3_2"]["parity_records_checked"] = int(n3 * H)
            out["trellis_3_2"]["parity_records_equal"] = eq3
            out["trellis_3_2"]["cpu_baseline"] = {
                "value": round(n3 * G / med, 1), "unit": "tokens/s", "cores": n_threads, "kind": kind,
                "ms_per_commit": round(med * 1e3, 1),
                "sample": "the whole 3/2 trellis commit (32 groups x 4 heads = 128 records) sealed by layer_seal from "
                          "the same ring bytes, groups split over %d threads; median of %d runs (%.3f s, spread "
                          "%.3f-%.3f s)" % (n_threads, CPU_RUNS, med, lo, hi),
                "runs": CPU_RUNS, "spread_tokens_per_s": [round(n3 * G / hi, 1), round(n3 * G / lo, 1)],
                "single_thread": {"value": round(st3 * G / med1, 1), "unit": "tokens/s",
                                  "ms_per_commit": round(med1 * n3 / st3 * 1e3, 1),
                                  "ms_per_record": round(med1 / (st3 * H) * 1e3, 2),
                                  "sample": "%d groups (%d records) on one thread, median of %d runs (%.3f s, spread "
                                            "%.3f-%.3f s), scaled to the 32-group commit" %
                                            (st3, st3 * H, CPU_RUNS, med1, lo1, hi1),
                                  "spread_tokens_per_s": [round(st3 * G / hi1, 1), round(st3 * G / lo1, 1)]}}
            out["trellis_3_2"]["cpu_baseline"].update(cpu_info(kind))

    # ---------------- C4: tq6_0 append + decode attention at 100K ----------------
    bodies = args.attn_bodies.split(",")
    if not args.no_attn and "4/4" in bodies:
        N = 100000
        B, commits = decode_schedule_B(lib, N)
        ctx = attention_context(lib, dev, stream, N, B, commits, 4, 4, 0)
        cfg4, L4, v4, n_body, tail, alg_bytes, copies = ctx
        n_q, n_head = 4, 16
        q = np.random.default_rng(4).standard_normal((n_q, n_head, D)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        qpos0 = N - n_q
        ms_a = time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args)
        gbs = alg_bytes / (ms_a * 1e-3) / 1e9
        # append of 4 positions (K and V of 4 heads), fused rotation + tq6_0, into the ring past N
        Ka, Va = inputs.kv_rows(4, H, D, seed=99)
        dKa, dVa = dev.put(Ka), dev.put(Va)
        app = lambda: lib.sjk_hip_layer_store(C.byref(v4), N, 4, dKa, dVa, 1, stream)  # noqa: E731
        ms_app, _ = timed(dev, stream, app, 50, 5)
        # the same call with (B, N, qpos0) in a device descriptor (sjk_hip_attend_dyn: plan kernel + fixed grid)
        desc = np.zeros(16, np.int32)
        desc[2], desc[3], desc[4] = B, N, qpos0
        d_desc = dev.put(desc)
        dyn_it = [0]

        def attend_dyn():
            v = copies[0][dyn_it[0] % len(copies[0])]
            dyn_it[0] += 1
            return lib.sjk_hip_attend_dyn(C.byref(v), d_desc, N, n_q, n_head, dq, 1.0 / 16.0, do, stream)

        sjk.check(attend_dyn(), "attend_dyn")
        ms_dyn, _ = timed(dev, stream, attend_dyn, args.attn_calls or max(50, args.steps) * len(copies[0]),
                          args.attn_warmup)
        sjk.check(lib.sjk_hip_attend(C.byref(copies[0][0]), B, N, qpos0, n_q, n_head, dq, 1.0 / 16.0, do, stream),
                  "attend")
        dev.hip.hipStreamSynchronize(stream)
        out["attention"] = {"workload": "configs[3]: N=100,000, B=%d (%d sealed groups), tq6_0 tail %d, fp16 sink 128, "
                                        "4/4 body, decode width 4, 16 query heads / 4 KV heads, D=256" % (B, n_body, tail),
                            "us_per_call": round(ms_a * 1e3, 2), "hbm_GBps": round(gbs, 1),
                            "algorithmic_bytes": int(alg_bytes), "target_us_60pct": 23.5,
                            "append_4pos_us": round(ms_app * 1e3, 2),
                            "attend_dyn_us": round(ms_dyn * 1e3, 2)}
        out["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                           "kernel": "attend4_kernel + attend3_combine (one sjk_hip_attend call, 4/4 body)"}
        # decode widths 1 and 5 and GQA 8:1 on the same context (20 and 32 rows per KV head: two 16-row jobs)
        got16 = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, D)
        sh_rep, sh_outs = time_shapes(lib, dev, stream, copies, B, N, D, H, alg_bytes - n_q * n_head * D * 6, gbs,
                                      (("width1", 1, 16), ("width5", 5, 16), ("gqa8_width4", 4, 32)), args)
        out["attention"]["shapes"] = sh_rep
        dev.upload(do, got16)
        # attention parity at full size on a few rows, and the CPU baseline on the same cache
        got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, D)
        if not args.no_cpu:
            clib, kind = cpu_lib(cabi)
            OL = oracle_layer_from_device(clib, cabi, dev, cfg4, L4, n_body)
            pairs = [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
            n_thr = cpu_threads()
            log("[bench] CPU baseline (%s): layer_attend_row for %d (row, head) pairs at N=100K on %d threads, "
                "%d runs" % (kind, len(pairs), n_thr, CPU_RUNS))
            ts = []
            for _ in range(CPU_RUNS):
                want, dt = oracle_attend(clib, cabi, OL, q, B, N, qpos0, pairs, n_thr)
                ts.append(dt)
            err = max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs)
            out["attention"]["parity_max_err_over_tol"] = round(err, 4)
            out["attention"]["shapes_parity_max_err_over_tol"] = shapes_parity(clib, cabi, OL, B, N, H, sh_outs)
            st_pairs = [(0, 0), (3, 15)]
            ts1 = [oracle_attend(clib, cabi, OL, q, B, N, qpos0, st_pairs, 1)[1] for _ in range(3)]
            med, lo, hi = spread(ts)
            med1, lo1, hi1 = spread(ts1)
            scale1 = len(pairs) / len(st_pairs)
            out["attention"]["cpu_baseline"] = {
                "us_per_call": round(med * 1e6, 1), "cores": n_thr, "kind": kind,
                "sample": "the whole call: %d (row, head) pairs of layer_attend_row at N=100K on %d threads; median of "
                          "%d runs (%.2f s, spread %.2f-%.2f s)" % (len(pairs), n_thr, CPU_RUNS, med, lo, hi),
                "runs": CPU_RUNS, "spread_us": [round(lo * 1e6, 1), round(hi * 1e6, 1)],
                "single_thread": {"us_per_call": round(med1 * scale1 * 1e6, 1),
                                  "sample": "%d pairs on one thread, median of 3 runs (%.2f s, spread %.2f-%.2f s), "
                                            "scaled to the 64-pair call" % (len(st_pairs), med1, lo1, hi1)}}
            out["attention"]["cpu_baseline"].update(cpu_info(kind))
            clib.layer_free(C.byref(OL))
        free_context(lib, dev, ctx)

    if not args.no_attn and "3/3t" in bodies:
        # the same schedule with the 3/3 trellis body of configs[4]
        N = 100000
        n_q, n_head = 4, 16
        qpos0 = N - n_q
        B, commits = decode_schedule_B(lib, N)
        q = np.random.default_rng(4).standard_normal((n_q, n_head, D)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        ctx = attention_context(lib, dev, stream, N, B, commits, 3, 3, 1)
        cfgt, Lt, vt, n_body, tail, alg_t, copies = ctx
        ms_t = time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args)
        # the same call through sjk_hip_attend_dyn (bounds in a device descriptor, fixed launch shape)
        desc = np.zeros(16, np.int32)
        desc[2], desc[3], desc[4] = B, N, qpos0
        d_desc = dev.put(desc)
        dyn_it = [0]

        def attend_dyn_t():
            v = copies[0][dyn_it[0] % len(copies[0])]
            dyn_it[0] += 1
            return lib.sjk_hip_attend_dyn(C.byref(v), d_desc, N, n_q, n_head, dq, 1.0 / 16.0, do, stream)

        sjk.check(attend_dyn_t(), "attend_dyn 3/3t")
        ms_tdyn, _ = timed(dev, stream, attend_dyn_t, args.attn_calls or max(50, args.steps) * len(copies[0]),
                           args.attn_warmup // 4)
        sjk.check(lib.sjk_hip_attend(C.byref(copies[0][0]), B, N, qpos0, n_q, n_head, dq, 1.0 / 16.0, do, stream),
                  "attend")
        dev.hip.hipStreamSynchronize(stream)
        gbs_t = alg_t / (ms_t * 1e-3) / 1e9
        out["attention_3_3t"] = {"workload": "N=100,000 as above with the 3/3 trellis body (records of %d bytes)" %
                                             Lt.lay.bytes, "us_per_call": round(ms_t * 1e3, 2),
                                 "hbm_GBps": round(gbs_t, 1), "algorithmic_bytes": int(alg_t),
                                 "attend_dyn_us": round(ms_tdyn * 1e3, 2)}
        got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, D)
        sh_rep, sh_outs = time_shapes(lib, dev, stream, copies, B, N, D, H, alg_t - n_q * n_head * D * 6, gbs_t,
                                      (("width5", 5, 16),), args)
        out["attention_3_3t"]["shapes"] = sh_rep
        if not args.no_cpu:
            OL = oracle_layer_from_device(orc, cabi, dev, cfgt, Lt, n_body)
            pairs = [(0, 0), (3, 15)]
            want, _ = oracle_attend(orc, cabi, OL, q, B, N, qpos0, pairs, 2)
            out["attention_3_3t"]["parity_max_err_over_tol"] = round(
                max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs), 4)
            out["attention_3_3t"]["shapes_parity_max_err_over_tol"] = shapes_parity(orc, cabi, OL, B, N, H, sh_outs)
            orc.layer_free(C.byref(OL))
        free_context(lib, dev, ctx)

    if not args.no_attn and "3/3s" in bodies:
        # configs[3]'s schedule with the 3/3 scalar body (token-major 3-bit sides), the kernel of the scalar bodies
        # other than 4/4
        N = 100000
        n_q, n_head = 4, 16
        qpos0 = N - n_q
        B, commits = decode_schedule_B(lib, N)
        q = np.random.default_rng(4).standard_normal((n_q, n_head, D)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        ctx = attention_context(lib, dev, stream, N, B, commits, 3, 3, 0)
        cfgs, Ls, vs_, n_body, tail, alg_s, copies = ctx
        ms_s = time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args)
        gbs_s = alg_s / (ms_s * 1e-3) / 1e9
        out["attention_3_3s"] = {"workload": "N=100,000 as above with the 3/3 scalar body (records of %d bytes)" %
                                             Ls.lay.bytes, "us_per_call": round(ms_s * 1e3, 2),
                                 "hbm_GBps": round(gbs_s, 1), "algorithmic_bytes": int(alg_s)}
        got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, D)
        sh_rep, sh_outs = time_shapes(lib, dev, stream, copies, B, N, D, H, alg_s - n_q * n_head * D * 6, gbs_s,
                                      (("width5", 5, 16),), args)
        out["attention_3_3s"]["shapes"] = sh_rep
        if not args.no_cpu:
            OL = oracle_layer_from_device(orc, cabi, dev, cfgs, Ls, n_body)
            pairs = [(0, 0), (3, 15)]
            want, _ = oracle_attend(orc, cabi, OL, q, B, N, qpos0, pairs, 2)
            out["attention_3_3s"]["parity_max_err_over_tol"] = round(
                max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs), 4)
            out["attention_3_3s"]["shapes_parity_max_err_over_tol"] = shapes_parity(orc, cabi, OL, B, N, H, sh_outs)
            orc.layer_free(C.byref(OL))
        free_context(lib, dev, ctx)

    # the other scalar bodies (4/3s ... 2/2s, not 4/4 or 3/3s; "d128": head dimension 128, 8 KV heads, 32 query
    # heads), same schedule and rotation, each timed and (with the CPU legs) checked on two (row, head) pairs
    for body in bodies:
        if args.no_attn or not re.fullmatch(r"[234]/[234]s(d128)?", body) or body == "3/3s" or body.startswith("4/4"):
            continue
        bk, bv, d128 = int(body[0]), int(body[2]), body.endswith("d128")
        N, d, h, n_q = 100000, (128 if d128 else D), (8 if d128 else H), 4
        n_head = 4 * h
        qpos0 = N - n_q
        B, commits = decode_schedule_B(lib, N)
        q = np.random.default_rng(4).standard_normal((n_q, n_head, d)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        ctx = attention_context(lib, dev, stream, N, B, commits, bk, bv, 0, d=d, h=h, n_head=n_head)
        cfgx, Lx, vx, n_body, tail, alg_x, copies = ctx
        ms_x = time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args)
        rep = {"record_bytes": int(Lx.lay.bytes), "us_per_call": round(ms_x * 1e3, 2),
               "hbm_GBps": round(alg_x / (ms_x * 1e-3) / 1e9, 1), "algorithmic_bytes": int(alg_x)}
        if not args.no_cpu:
            got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, d)
            OL = oracle_layer_from_device(orc, cabi, dev, cfgx, Lx, n_body)
            pairs = [(0, 0), (3, n_head - 1)]
            want, _ = oracle_attend(orc, cabi, OL, q, B, N, qpos0, pairs, 2)
            rep["parity_max_err_over_tol"] = round(
                max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs), 4)
            orc.layer_free(C.byref(OL))
        out.setdefault("attention_scalar_bodies", {
            "workload": "N=100,000 as configs[3] (decode width 4, GQA 4:1) with other scalar bodies; d128: head "
                        "dimension 128, 8 KV heads, 32 query heads"})[body] = rep
        free_context(lib, dev, ctx)

    if not args.no_attn and "3/3td128" in bodies:
        # the 3/3 trellis body at head dimension 128 (8 KV heads, 32 query heads, width 4): the trellis kernel's
        # D = 128 instance (not in the default set)
        N, d, h, n_q, n_head = 100000, 128, 8, 4, 32
        qpos0 = N - n_q
        B, commits = decode_schedule_B(lib, N)
        q = np.random.default_rng(4).standard_normal((n_q, n_head, d)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        ctx = attention_context(lib, dev, stream, N, B, commits, 3, 3, 1, d=d, h=h, n_head=n_head)
        cfgt, Lt, vt, n_body, tail, alg_t, copies = ctx
        ms_t = time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args)
        out["attention_3_3t_d128"] = {"workload": "N=100,000 as above with head dimension 128: 8 KV heads, 32 query "
                                                  "heads (GQA 4:1), width 4, 3/3 trellis body (records of %d bytes)" %
                                                  Lt.lay.bytes, "us_per_call": round(ms_t * 1e3, 2),
                                      "hbm_GBps": round(alg_t / (ms_t * 1e-3) / 1e9, 1), "algorithmic_bytes": int(alg_t)}
        if not args.no_cpu:
            got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, d)
            OL = oracle_layer_from_device(orc, cabi, dev, cfgt, Lt, n_body)
            pairs = [(0, 0), (3, 31)]
            want, _ = oracle_attend(orc, cabi, OL, q, B, N, qpos0, pairs, 2)
            out["attention_3_3t_d128"]["parity_max_err_over_tol"] = round(
                max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs), 4)
            orc.layer_free(C.byref(OL))
        free_context(lib, dev, ctx)

    if not args.no_attn and "4/4d128" in bodies:
        # the 4/4 body at head dimension 128 (8 KV heads, 32 query heads: GQA 4:1, width 4), the common decode
        # shape of D = 128 models; same schedule, same rotation over device copies
        N, d, h, n_q, n_head = 100000, 128, 8, 4, 32
        qpos0 = N - n_q
        B, commits = decode_schedule_B(lib, N)
        q = np.random.default_rng(4).standard_normal((n_q, n_head, d)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        ctx = attention_context(lib, dev, stream, N, B, commits, 4, 4, 0, d=d, h=h, n_head=n_head)
        cfgd, Ld, vd, n_body, tail, alg_d, copies = ctx
        ms_d = time_attention(lib, dev, stream, copies, B, N, qpos0, dq, do, n_q, n_head, args)
        desc = np.zeros(16, np.int32)
        desc[2], desc[3], desc[4] = B, N, qpos0
        d_desc = dev.put(desc)
        dyn_it = [0]

        def attend_dyn_d():
            v = copies[0][dyn_it[0] % len(copies[0])]
            dyn_it[0] += 1
            return lib.sjk_hip_attend_dyn(C.byref(v), d_desc, N, n_q, n_head, dq, 1.0 / 16.0, do, stream)

        sjk.check(attend_dyn_d(), "attend_dyn d128")
        ms_ddyn, _ = timed(dev, stream, attend_dyn_d, args.attn_calls or max(50, args.steps) * len(copies[0]),
                           args.attn_warmup // 4)
        sjk.check(lib.sjk_hip_attend(C.byref(copies[0][0]), B, N, qpos0, n_q, n_head, dq, 1.0 / 16.0, do, stream),
                  "attend")
        dev.hip.hipStreamSynchronize(stream)
        gbs_d = alg_d / (ms_d * 1e-3) / 1e9
        out["attention_d128"] = {"workload": "N=100,000 as above with head dimension 128: 8 KV heads, 32 query heads "
                                             "(GQA 4:1), width 4, 4/4 body (records of %d bytes)" % Ld.lay.bytes,
                                 "us_per_call": round(ms_d * 1e3, 2),
                                 "hbm_GBps": round(gbs_d, 1), "algorithmic_bytes": int(alg_d),
                                 "attend_dyn_us": round(ms_ddyn * 1e3, 2)}
        got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, d)
        # GQA 8:1 (64 query heads over the 8 KV heads, width 4: 32 rows per KV head, two 16-row jobs)
        sh_rep, sh_outs = time_shapes(lib, dev, stream, copies, B, N, d, h, alg_d - n_q * n_head * d * 6, gbs_d,
                                      (("gqa8_width4", 4, 64),), args)
        out["attention_d128"]["shapes"] = sh_rep
        if not args.no_cpu:
            OL = oracle_layer_from_device(orc, cabi, dev, cfgd, Ld, n_body)
            pairs = [(0, 0), (3, 31), (1, 13), (2, 22)]
            want, _ = oracle_attend(orc, cabi, OL, q, B, N, qpos0, pairs, 4)
            out["attention_d128"]["parity_max_err_over_tol"] = round(
                max(float(np.max(np.abs(got[p] - want[p]) / (1e-3 + 1e-3 * np.abs(want[p])))) for p in pairs), 4)
            out["attention_d128"]["shapes_parity_max_err_over_tol"] = shapes_parity(orc, cabi, OL, B, N, h, sh_outs)
            orc.layer_free(C.byref(OL))
        free_context(lib, dev, ctx)

    # ---------------- C5: 16 layers x 8 sequences on one paged pool, 3/3 trellis ----------------
    if not args.no_pool:
        import pool_stress
        ps, rep = pool_stress.run(lib, dev, inputs.kv_rows, steps=args.pool_steps, log=log)
        rep["workload"] = ("configs[4]: 16 layers, 4 KV heads, D=256, 3/3 trellis body, 8 sequences on one paged "
                           "record pool, seeded prompts 8K-32K, %d decode rounds at width 4 (16 query heads), tail "
                           "4096 / tail_max 8192, one truncation into the body and one state save/restore half-way; "
                           "a round = every sequence's begin_ubatch (+ commit when due), append of 4 positions to 16 "
                           "layers, decode attention in 16 layers" % ps.steps)
        if not args.no_cpu:
            import pool_check
            log("[bench] C5: sampled CPU checks (records re-sealed by the oracle, attention rows)")
            chk = {}
            last = lambda s: (ps.seqs[s].pol.B - S) // G - 1  # noqa: E731
            recs = [(0, 0, last(0)), (1, 15, 0), (5, 7, last(5))]
            chk["records_checked"] = len(recs) * H
            chk["records_equal"] = sum(pool_check.check_records(orc, ps, s, il, [g]) for s, il, g in recs)
            chk["attention_max_err_over_tol"] = round(max(
                pool_check.check_attention(orc, ps, s, il, [(0, 0), (3, 15)]) for s, il in ((0, 0), (7, 15))), 4)
            chk["sample"] = ("records (seq, layer, group) %s re-sealed on the CPU from the run's input rows; attention "
                             "rows (0,0), (3,15) of (seq 0, layer 0) and (seq 7, layer 15) vs the oracle loop" % recs)
            rep["checks"] = chk
        ps.free()
        # the same prompts with the reference's chunked drain: a decode-sized ubatch seals at most flush_chunk
        # groups of every layer and leaves the rest draining (sj_kvarn.h:1329-1349), so that a commit's 16-layer
        # trellis seal is spread over the following rounds instead of landing in one
        nfc = max(2, ps.steps // 2)
        log("[bench] C5 with flush_chunk = 1: prefill and %d decode rounds" % nfc)
        psf = pool_stress.PoolStress(lib, dev, inputs.kv_rows, steps=nfc, flush_chunk=1, log=log)
        psf.prefill()
        Bp = [int(sq.pol.B) for sq in psf.seqs]
        dfc, wfc = psf.decode(nfc)
        fc = {"workload": "configs[4]'s prompts and decode batch with flush_chunk = 1 (every decode round seals at most "
                          "one group of each of the 16 layers while a commit drains), %d rounds, no truncation or "
                          "save" % nfc,
              "rounds": int(len(dfc)), "commits": psf.stats["commits"],
              "groups_sealed_in_decode": int(sum((int(sq.pol.B) - b) // G for sq, b in zip(psf.seqs, Bp))),
              "device_ms_per_round": {"mean": round(float(dfc.mean()), 4), "median": round(float(np.median(dfc)), 4),
                                      "p99": round(float(np.percentile(dfc, 99)), 4), "max": round(float(dfc.max()), 4)}}
        if not args.no_cpu:
            import pool_check
            drained = [(s, 15, (int(psf.seqs[s].pol.B) - S) // G - 1) for s in range(psf.n_seq)
                       if int(psf.seqs[s].pol.B) > Bp[s]][:2]
            fc["records_checked"] = len(drained) * H
            fc["records_equal"] = sum(pool_check.check_records(orc, psf, s, il, [g]) for s, il, g in drained)
            fc["sample"] = "the last group each of two sequences sealed during the drain, layer 15: %s" % drained
        rep["flush_chunk_1"] = fc
        psf.free()
        out["pool_stress"] = rep

    if args.copy_calib:
        nb = args.copy_calib << 20
        src, dst = dev.alloc(nb), dev.alloc(nb, zero=False)
        for _ in range(4):
            dev._ck(dev.hip.hipMemcpyAsync(dst, src, nb, dev.D2D, stream), "hipMemcpyAsync")
        dev.hip.hipStreamSynchronize(stream)
        out["copy_calib_bytes"] = nb

    for ly in (L, L3):
        if ly is not None:
            lib.sj_kvarn_layer_free(C.byref(ly))
    dev.free_all()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
