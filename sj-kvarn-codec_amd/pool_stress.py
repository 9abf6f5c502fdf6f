"""Per-sequence cache stress on one GPU: many layers and sequences on one paged record pool.

The workload of the reference's per-sequence API (sj_kvarn.h:1645-1809) at engine scale: every sequence
gets a seeded random-length prompt, stored in 512-position ubatches, then `steps` decode rounds at width
`width`. A decode round is, for every sequence, sj_kvarn_seq_begin_ubatch (the adaptive-tail policy,
which seals [B, B_pending) of all layers in one launch when a commit is due, sj_kvarn.h:1332-1355,
1760-1770), the append of `width` positions to every layer (sjk_hip_seq_store: fused Hadamard + tq6_0
staging) and decode attention for `width` query rows in every layer (sjk_hip_seq_attend). Mid-run one
sequence is truncated (sj_kvarn_seq_truncate, sj_kvarn.h:1794-1804) and another is saved to a state
stream, freed, re-created on the pool and restored from it (sj_kvarn.h:1811-2034).

Everything runs on the null stream of the current device; commits are enqueued there in stream order
(sjk_hip_seq_begin_ubatch: no host wait). The time of a round is taken with HIP events around it (device time,
commits included) and with the host clock. The state save of the mid-run check is asynchronous
(sjk_hip_seq_state_write_begin / _finish): the rounds go on while the stream is copied out, and the restore
(sjk_hip_seq_state_read_begin / _finish) runs while the other sequences decode.

Input rows are a pure function of (position, sequence, layer, generation): position p reads row
(p + c) % R of a pool of R seeded rows held on the device (R + 512 rows, so that any ubatch of up to 512
positions is one contiguous slice), with c = 977 s + 131 l + 1013 gen; a sequence's generation is raised
at its truncation, so the positions stored again after a cut differ from the ones cut away. `rows()`
rebuilds any position's input on the host for a checker.
"""
import ctypes as C
import time

import numpy as np

import sjk

R_ROWS = 8192          # distinct synthetic positions
UB_MAX = 512           # prefill ubatch


class PoolStress:
    def __init__(self, lib, dev, kv_rows, n_layers=16, n_seq=8, H=4, D=256, bk=3, bv=3, body=sjk.BODY_TRELLIS,
                 prompt=(8192, 32768), steps=2048, width=4, n_head=16, seed=5, tail=4096, tail_max=8192,
                 batched=True, flush_chunk=0, log=print):
        """kv_rows(n, H, D, seed) -> (K, V) float32 [n][H][D]: the seeded row generator"""
        self.lib, self.dev, self.log = lib, dev, log
        self.n_layers, self.n_seq, self.H, self.D, self.width, self.n_head = n_layers, n_seq, H, D, width, n_head
        self.steps = steps
        self.scale = 1.0 / float(np.sqrt(D))
        rng = np.random.default_rng(seed)
        self.prompt = [int(x) for x in rng.integers(prompt[0], prompt[1] + 1, n_seq)]
        n_ctx = max(self.prompt) + steps * width + 1024
        self.cfg = lib.sj_kvarn_config_default(D, H, n_ctx, UB_MAX)
        self.cfg.bits_k, self.cfg.bits_v, self.cfg.body = bk, bv, body
        self.cfg.tail, self.cfg.tail_max, self.cfg.flush_chunk = tail, tail_max, flush_chunk
        self.S, self.G = int(self.cfg.sink), int(self.cfg.group)
        groups = (n_ctx - self.S + self.G - 1) // self.G
        self.pool = sjk.Pool()
        sjk.check(lib.sj_kvarn_pool_init(C.byref(self.pool), C.byref(self.cfg), n_layers, n_seq * groups), "pool_init")
        self.seqs = []
        for _ in range(n_seq):
            s = sjk.Seq()
            sjk.check(lib.sj_kvarn_seq_init(C.byref(s), C.byref(self.cfg), n_layers, C.byref(self.pool)), "seq_init")
            self.seqs.append(s)
        self.gen = [0] * n_seq               # generation of the rows stored from gen_from[s] on
        self.gen_from = [0] * n_seq
        K, V = kv_rows(R_ROWS, H, D, seed + 1000)
        self.Kh = np.concatenate([K, K[:UB_MAX]])
        self.Vh = np.concatenate([V, V[:UB_MAX]])
        self.dK, self.dV = dev.put(self.Kh), dev.put(self.Vh)
        self.row_bytes = H * D * 4
        q = rng.standard_normal((n_seq, width, n_head, D)).astype(np.float32)
        self.q = q
        self.dq = [dev.put(q[s]) for s in range(n_seq)]
        self.dout = [dev.alloc(q[s].nbytes) for s in range(n_seq)]
        self.stats = {"commits": 0, "commit_wall_ms": 0.0}
        # decode batch: one job per sequence (sjk_hip_seq_store_batch / sjk_hip_seq_attend_batch per layer)
        self.batched = batched
        self.jobs = (sjk.SeqJob * n_seq)()
        for s in range(n_seq):
            self._bind_job(s)
            self.jobs[s].d_q, self.jobs[s].d_out = self.dq[s].value, self.dout[s].value

    def _bind_job(self, s):
        self.jobs[s].seq = C.pointer(self.seqs[s])

    # ---- inputs ------------------------------------------------------------------------------------
    def _start(self, s, il, p0, gen):
        return (p0 + 977 * s + 131 * il + 1013 * gen) % R_ROWS

    def rows(self, s, il, p0, n):
        """host copy of the K and V rows the run stored for positions [p0, p0 + n) of (sequence, layer)"""
        K = np.empty((n, self.H, self.D), np.float32)
        V = np.empty_like(K)
        for i in range(n):
            p = p0 + i
            g = self.gen[s] if p >= self.gen_from[s] else 0
            r = self._start(s, il, p, g)
            K[i], V[i] = self.Kh[r], self.Vh[r]
        return K, V

    # ---- one ubatch of one sequence ------------------------------------------------------------------
    def _begin(self, s, pos0, n):
        seq = self.seqs[s]
        B0 = seq.pol.B
        t0 = time.perf_counter()
        sjk.check(self.lib.sjk_hip_seq_begin_ubatch(C.byref(seq), pos0, n, None), "sjk_hip_seq_begin_ubatch")
        if seq.pol.B != B0:
            self.stats["commits"] += 1
            self.stats["commit_wall_ms"] += (time.perf_counter() - t0) * 1e3

    def _store(self, s, pos0, n):
        seq = self.seqs[s]
        g = self.gen[s] if pos0 >= self.gen_from[s] else 0
        for il in range(self.n_layers):
            off = self._start(s, il, pos0, g) * self.row_bytes
            rc = self.lib.sjk_hip_seq_store(C.byref(seq), il, pos0, n, C.c_void_p(self.dK.value + off),
                                            C.c_void_p(self.dV.value + off), 1, None)
            sjk.check(rc, "sjk_hip_seq_store")

    def attend(self, s, il, out=None):
        """decode attention of sequence s, layer il for the last `width` positions (rotated queries)"""
        seq = self.seqs[s]
        rc = self.lib.sjk_hip_seq_attend(C.byref(seq), il, seq.n - self.width, self.width, self.n_head, self.dq[s],
                                         self.scale, out if out is not None else self.dout[s], None)
        sjk.check(rc, "sjk_hip_seq_attend")

    # ---- phases ------------------------------------------------------------------------------------
    def prefill(self):
        t0 = time.perf_counter()
        for s in range(self.n_seq):
            P = self.prompt[s]
            for p0 in range(0, P, UB_MAX):
                n = min(UB_MAX, P - p0)
                self._begin(s, p0, n)
                self._store(s, p0, n)
        self.dev.sync()
        return time.perf_counter() - t0

    def decode(self, rounds, events=True, active=None, until=None):
        """up to `rounds` decode rounds over the sequences `active` (default: all); stops after the round in which
        until() becomes true. Returns per-round (device ms, host ms) arrays of the rounds run."""
        dev, hip = self.dev, self.dev.hip
        active = list(range(self.n_seq)) if active is None else list(active)
        ev = [dev.event() for _ in range(rounds + 1)] if events else None
        wall = np.zeros(rounds)
        done = rounds
        for r in range(rounds):
            t0 = time.perf_counter()
            if events:
                dev._ck(hip.hipEventRecord(ev[r], None), "hipEventRecord")
            if self.batched:
                self._round_batched(active)
            else:
                for s in active:
                    pos = self.seqs[s].n
                    self._begin(s, pos, self.width)
                    self._store(s, pos, self.width)
                    for il in range(self.n_layers):
                        self.attend(s, il)
            wall[r] = time.perf_counter() - t0
            if until is not None and until():
                done = r + 1
                break
        if events:
            dev._ck(hip.hipEventRecord(ev[done], None), "hipEventRecord")
            dev._ck(hip.hipEventSynchronize(ev[done]), "hipEventSynchronize")
            devms = np.array([dev.elapsed_ms(ev[r], ev[r + 1]) for r in range(done)])
            for e in ev:
                hip.hipEventDestroy(e)
        else:
            dev.sync()
            devms = None
        return devms, wall[:done] * 1e3

    def _round_batched(self, active):
        """a decode round as an engine batches it: every sequence's policy step, then per layer one
        launch that appends all sequences' positions and one that runs all their attention"""
        lib, w = self.lib, self.width
        jobs = (sjk.SeqJob * len(active))()
        pos = []
        for k, s in enumerate(active):
            p = self.seqs[s].n
            self._begin(s, p, w)
            pos.append((p, self.gen[s] if p >= self.gen_from[s] else 0))
            jobs[k] = self.jobs[s]
        for il in range(self.n_layers):
            for k, s in enumerate(active):
                p, g = pos[k]
                off = self._start(s, il, p, g) * self.row_bytes
                jobs[k].pos0 = p
                jobs[k].d_k = self.dK.value + off
                jobs[k].d_v = self.dV.value + off
            sjk.check(lib.sjk_hip_seq_store_batch(jobs, len(active), il, w, 1, None), "sjk_hip_seq_store_batch")
            sjk.check(lib.sjk_hip_seq_attend_batch(jobs, len(active), il, w, self.n_head, self.scale, None),
                      "sjk_hip_seq_attend_batch")

    def truncate(self, s, back):
        """cut sequence s (once) to n - back positions; returns (requested, kept) position counts"""
        if self.gen[s]:
            raise RuntimeError("one truncation per sequence: rows() keeps a single generation boundary")
        seq = self.seqs[s]
        want = seq.n - back
        r = self.lib.sj_kvarn_seq_truncate(C.byref(seq), want)
        if r == sjk.NO_POS:
            raise RuntimeError("sj_kvarn_seq_truncate refused position %d" % want)
        self.gen[s], self.gen_from[s] = 1, int(r)
        return want, int(r)

    def state_bytes(self, s):
        seq = self.seqs[s]
        n = self.lib.sj_kvarn_seq_state_size(C.byref(seq))
        buf = np.zeros(n, np.uint8)
        w = C.c_size_t(0)
        sjk.check(self.lib.sj_kvarn_seq_state_write(C.byref(seq), buf.ctypes.data, n, C.byref(w)), "seq_state_write")
        assert w.value == n
        return buf

    def save_async(self, s, rounds_max):
        """the asynchronous save of sequence s while decode rounds of every sequence (s included) go on; returns
        (stream, begin ms, wall ms to the stream's end, per-round device ms, host ms of the rounds run meanwhile)"""
        seq = self.seqs[s]
        n = self.lib.sj_kvarn_seq_state_size(C.byref(seq))
        buf = np.zeros(n, np.uint8)
        t0 = time.perf_counter()
        sjk.check(self.lib.sjk_hip_seq_state_write_begin(C.byref(seq), buf.ctypes.data, n), "state_write_begin")
        t1 = time.perf_counter()
        dms, wms = self.decode(rounds_max, until=lambda: self.lib.sjk_hip_seq_state_poll(C.byref(self.seqs[s])) == 1)
        w = C.c_size_t(0)
        sjk.check(self.lib.sjk_hip_seq_state_finish(C.byref(seq), C.byref(w)), "state_finish")
        t2 = time.perf_counter()
        assert w.value == n
        return buf, (t1 - t0) * 1e3, (t2 - t0) * 1e3, dms, wms

    def restore_async(self, s, buf, rounds_max):
        """free sequence s, re-create it on the pool and restore `buf` into it while the other sequences decode;
        returns (wall ms, per-round device ms, host ms of the rounds run meanwhile)"""
        self.lib.sj_kvarn_seq_free(C.byref(self.seqs[s]))
        seq = sjk.Seq()
        sjk.check(self.lib.sj_kvarn_seq_init(C.byref(seq), C.byref(self.cfg), self.n_layers, C.byref(self.pool)),
                  "seq_init")
        self.seqs[s] = seq
        t0 = time.perf_counter()
        sjk.check(self.lib.sjk_hip_seq_state_read_begin(C.byref(seq), buf.ctypes.data, buf.nbytes), "state_read_begin")
        others = [k for k in range(self.n_seq) if k != s]
        dms, wms = self.decode(rounds_max, active=others,
                               until=lambda: self.lib.sjk_hip_seq_state_poll(C.byref(seq)) == 1)
        sjk.check(self.lib.sjk_hip_seq_state_finish(C.byref(seq), None), "state_finish")
        t1 = time.perf_counter()
        self._bind_job(s)
        return (t1 - t0) * 1e3, dms, wms

    def free(self):
        for s in self.seqs:
            self.lib.sj_kvarn_seq_free(C.byref(s))
        self.lib.sj_kvarn_pool_free(C.byref(self.pool))
        self.seqs = []


def run(lib, dev, kv_rows, truncate_round=None, trunc_back=10000, save_seq=1, trunc_seq=0, log=print, **kw):
    """The whole stress run: prefill, decode rounds with the truncation and the state save/restore at
    `truncate_round` (default: half-way). Returns (PoolStress, report dict); the caller frees it."""
    ps = PoolStress(lib, dev, kv_rows, log=log, **kw)
    rep = {"prompts": ps.prompt, "batched": ps.batched}
    log("[pool] prefill of %d sequences x %d layers (%d positions)" % (ps.n_seq, ps.n_layers, sum(ps.prompt)))
    rep["prefill_s"] = round(ps.prefill(), 3)
    half = ps.steps // 2 if truncate_round is None else truncate_round
    log("[pool] %d decode rounds" % half)
    d1, w1 = ps.decode(half)
    # truncation of one sequence, state save / restore of another
    B_before, n_before = int(ps.seqs[trunc_seq].pol.B), int(ps.seqs[trunc_seq].n)
    want, kept = ps.truncate(trunc_seq, min(trunc_back, ps.seqs[trunc_seq].n - ps.S - 1))
    rep["truncate"] = {"seq": trunc_seq, "n_before": n_before, "B_before": B_before, "to": want, "kept": kept,
                       "B_after": int(ps.seqs[trunc_seq].pol.B)}
    dev.sync()
    before = dev.alloc(ps.q[save_seq].nbytes)
    after = dev.alloc(ps.q[save_seq].nbytes)
    ps.attend(save_seq, ps.n_layers - 1, before)
    # the synchronous stream of this moment (the reference for the asynchronous one)
    t0 = time.perf_counter()
    want = ps.state_bytes(save_seq)
    t_write = time.perf_counter() - t0
    left = ps.steps - half
    log("[pool] asynchronous save of sequence %d (%d bytes) while every sequence decodes" % (save_seq, want.nbytes))
    saved, begin_ms, save_ms, ds, wsv = ps.save_async(save_seq, left)
    left -= len(ds)
    log("[pool] asynchronous restore of sequence %d while the other %d decode" % (save_seq, ps.n_seq - 1))
    restore_ms, dr, wr = ps.restore_async(save_seq, saved, max(left, 1))
    left -= len(dr)
    ps.attend(save_seq, ps.n_layers - 1, after)
    again = ps.state_bytes(save_seq)
    nb = ps.q[save_seq].nbytes

    def st(a):
        return {"mean": round(float(a.mean()), 4), "max": round(float(a.max()), 4)} if len(a) else {}

    rep["save_restore"] = {"seq": save_seq, "state_bytes": int(saved.nbytes),
                           "write_ms": round(t_write * 1e3, 1),
                           "async_save": {"begin_ms": round(begin_ms, 2), "wall_ms": round(save_ms, 1),
                                          "rounds_during": len(ds), "device_ms_per_round_during": st(ds),
                                          "stream_equal_sync": bool(np.array_equal(saved, want))},
                           "async_restore": {"wall_ms": round(restore_ms, 1), "rounds_during": len(dr),
                                             "sequences_decoding": ps.n_seq - 1,
                                             "device_ms_per_round_during": st(dr)},
                           "stream_equal": bool(np.array_equal(saved, again)),
                           "attention_equal": bool(np.array_equal(dev.get(before, nb, np.uint8),
                                                                  dev.get(after, nb, np.uint8)))}
    dev.free(before)
    dev.free(after)
    log("[pool] %d decode rounds" % left)
    d2, w2 = ps.decode(left) if left > 0 else (np.zeros(0), np.zeros(0))
    dms, wms = np.concatenate([d1, ds, dr, d2]), np.concatenate([w1, wsv, wr, w2])
    rep["rounds"] = int(len(dms))
    rep["device_ms_per_round"] = {"mean": round(float(dms.mean()), 4), "median": round(float(np.median(dms)), 4),
                                  "p99": round(float(np.percentile(dms, 99)), 4), "max": round(float(dms.max()), 4)}
    rep["host_ms_per_round"] = {"mean": round(float(wms.mean()), 4), "median": round(float(np.median(wms)), 4)}
    rep["commits"] = ps.stats["commits"]
    rep["commit_wall_ms_total"] = round(ps.stats["commit_wall_ms"], 2)
    rep["final_positions"] = [int(s.n) for s in ps.seqs]
    rep["final_B"] = [int(s.pol.B) for s in ps.seqs]
    rep["pool_blocks_free"] = int(ps.pool.n_free)
    return ps, rep
