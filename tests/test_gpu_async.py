"""Commits and state transfers that do not stop the device (no counterpart in the reference's C API; its README
plans both: the seal "can run ahead of this ubatch's K/V writes, or on a side stream", README.md:351-352, and the
state save as "device-to-host copies overlapped with decoding", README.md:609).

  * sjk_hip_seq_begin_ubatch enqueues the commit on the caller's stream and returns: a sequence built that way on a
    non-blocking stream equals, byte for byte (state stream) and bit for bit (attention), one built with the drop-in
    sj_kvarn_seq_begin_ubatch, which now waits for its own seal only;
  * one sequence commits (drop-in calls, host-synchronous) while another decodes from a second host thread on its
    own stream: both equal the same work done serially;
  * sjk_hip_seq_state_write_begin / _read_begin / _poll / _finish: a save taken while another sequence decodes and
    the saved one keeps growing equals the synchronous stream of the same moment; a restore made while another
    sequence decodes gives the same stream and the same attention; a damaged stream is refused at _finish with the
    target untouched; a second transfer on a sequence with one in flight is refused.
"""
import ctypes as C
import sys
import threading
import time

import numpy as np
import pytest

import cabi
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

pytestmark = pytest.mark.gpu
D, H, NL, N_HEAD, W = 128, 2, 2, 8, 4


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.fixture(scope="module")
def dev():
    d = sjk.Device()
    d.hip.hipStreamCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
    yield d
    d.free_all()


def nonblocking_stream(dev):
    s = C.c_void_p()
    dev._ck(dev.hip.hipStreamCreateWithFlags(C.byref(s), 1), "hipStreamCreateWithFlags")
    return s


def config(lib, bk=3, bv=3, body=1):
    cfg = lib.sj_kvarn_config_default(D, H, 8192, 256)
    cfg.bits_k, cfg.bits_v, cfg.body, cfg.tail, cfg.tail_max = bk, bv, body, 256, 512
    return cfg


class Rows:
    """device rows [n][H][D] (K and V) and queries, fixed for the whole test: no buffer is freed while work runs"""

    def __init__(self, dev, n, seed):
        K, V = inputs.kv_rows(n, H, D, seed=seed)
        self.dK, self.dV = dev.put(K), dev.put(V)
        self.row = H * D * 4
        q = np.random.default_rng(seed + 1).standard_normal((W, N_HEAD, D)).astype(np.float32)
        self.nq = q.nbytes
        self.dq = dev.put(q)

    def k(self, p):
        return C.c_void_p(self.dK.value + p * self.row)

    def v(self, p):
        return C.c_void_p(self.dV.value + p * self.row)


def new_seq(lib, cfg, pool=None):
    s = sjk.Seq()
    sjk.check(lib.sj_kvarn_seq_init(C.byref(s), C.byref(cfg), NL, C.byref(pool) if pool is not None else None),
              "seq_init")
    return s


def new_pool(lib, cfg, blocks=80):
    p = sjk.Pool()
    sjk.check(lib.sj_kvarn_pool_init(C.byref(p), C.byref(cfg), NL, blocks), "pool_init")
    return p


def step(lib, s, rows, p0, n, stream, async_commit):
    """one ubatch of positions [p0, p0 + n): the policy step (commit when due), then the stores of every layer"""
    if async_commit:
        sjk.check(lib.sjk_hip_seq_begin_ubatch(C.byref(s), p0, n, stream), "sjk_hip_seq_begin_ubatch")
    else:
        sjk.check(lib.sj_kvarn_seq_begin_ubatch(C.byref(s), p0, n), "sj_kvarn_seq_begin_ubatch")
    for il in range(NL):
        sjk.check(lib.sjk_hip_seq_store(C.byref(s), il, p0, n, rows.k(p0), rows.v(p0), 1, stream), "seq_store")


def attend(lib, s, rows, out, stream, il=NL - 1):
    sjk.check(lib.sjk_hip_seq_attend(C.byref(s), il, s.n - W, W, N_HEAD, rows.dq, 0.0625, out, stream), "attend")


def grow(lib, dev, s, rows, n_prompt, rounds, stream, async_commit, outs=None):
    """prefill in 256-position ubatches, then `rounds` decode rounds of W positions (attention into outs[r])"""
    for p0 in range(0, n_prompt, 256):
        step(lib, s, rows, p0, min(256, n_prompt - p0), stream, async_commit)
    for r in range(rounds):
        step(lib, s, rows, s.n, W, stream, async_commit)
        if outs is not None:
            attend(lib, s, rows, outs[r], stream)


def stream_bytes(lib, s):
    n = lib.sj_kvarn_seq_state_size(C.byref(s))
    buf = np.zeros(n, np.uint8)
    w = C.c_size_t(0)
    sjk.check(lib.sj_kvarn_seq_state_write(C.byref(s), buf.ctypes.data, n, C.byref(w)), "state_write")
    assert w.value == n
    return buf


def test_stream_ordered_commit_equals_the_dropin_commit(lib, dev):
    cfg = config(lib)
    rows = Rows(dev, 3000, seed=7)
    pools = [new_pool(lib, cfg), new_pool(lib, cfg)]
    seqs = [new_seq(lib, cfg, pools[0]), new_seq(lib, cfg, pools[1])]
    st = nonblocking_stream(dev)
    rounds = 120
    outs = [[dev.alloc(rows.nq) for _ in range(rounds)] for _ in range(2)]
    try:
        grow(lib, dev, seqs[0], rows, 2400, rounds, st, False, outs[0])     # drop-in commits, stores on st
        dev.hip.hipStreamSynchronize(st)
        grow(lib, dev, seqs[1], rows, 2400, rounds, st, True, outs[1])      # commits enqueued on st, no wait
        dev.hip.hipStreamSynchronize(st)
        assert seqs[0].pol.B == seqs[1].pol.B and seqs[0].pol.B >= 2048     # several commits on the way
        assert np.array_equal(stream_bytes(lib, seqs[0]), stream_bytes(lib, seqs[1]))
        for r in range(rounds):
            assert np.array_equal(dev.get(outs[0][r], rows.nq, np.uint32), dev.get(outs[1][r], rows.nq, np.uint32)), r
    finally:
        dev.hip.hipStreamDestroy(st)
        for s in seqs:
            lib.sj_kvarn_seq_free(C.byref(s))
        for p in pools:
            lib.sj_kvarn_pool_free(C.byref(p))


def test_commit_while_another_sequence_decodes_on_another_thread(lib, dev):
    """thread 0 decodes sequence A (stores, stream-ordered commits, attention) on its stream; thread 1 prefills
    sequence B with drop-in commits (host-synchronous, waiting for B's seal only) on another stream. Each result
    equals the same sequence's work done alone."""
    cfg = config(lib)
    rows_a, rows_b = Rows(dev, 3200, seed=11), Rows(dev, 3200, seed=12)
    rounds = 150

    def run_pair(concurrent):
        pools = [new_pool(lib, cfg), new_pool(lib, cfg)]
        a, b = new_seq(lib, cfg, pools[0]), new_seq(lib, cfg, pools[1])
        sa, sb = nonblocking_stream(dev), nonblocking_stream(dev)
        outs = [dev.alloc(rows_a.nq) for _ in range(rounds)]
        grow(lib, dev, a, rows_a, 1800, 0, sa, True)                        # A's context first
        dev.hip.hipStreamSynchronize(sa)
        errors = []
        gate = threading.Barrier(2) if concurrent else None

        def decode_a():
            try:
                if gate:
                    gate.wait()
                for r in range(rounds):
                    step(lib, a, rows_a, a.n, W, sa, True)
                    attend(lib, a, rows_a, outs[r], sa)
                dev.hip.hipStreamSynchronize(sa)
            except Exception as e:  # noqa: BLE001
                errors.append(("A", repr(e)))

        def prefill_b():
            try:
                if gate:
                    gate.wait()
                grow(lib, dev, b, rows_b, 3000, 0, sb, False)
                dev.hip.hipStreamSynchronize(sb)
            except Exception as e:  # noqa: BLE001
                errors.append(("B", repr(e)))

        if concurrent:
            ths = [threading.Thread(target=decode_a), threading.Thread(target=prefill_b)]
            for t in ths:
                t.start()
            for t in ths:
                t.join()
        else:
            decode_a()
            prefill_b()
        assert not errors, errors
        got = [dev.get(o, rows_a.nq, np.uint32) for o in outs]
        res = (got, stream_bytes(lib, a), stream_bytes(lib, b), int(b.pol.B))
        for st in (sa, sb):
            dev.hip.hipStreamDestroy(st)
        for s in (a, b):
            lib.sj_kvarn_seq_free(C.byref(s))
        for p in pools:
            lib.sj_kvarn_pool_free(C.byref(p))
        for o in outs:
            dev.free(o)
        return res

    alone = run_pair(False)
    both = run_pair(True)
    assert alone[3] >= 2048                                                 # B committed several times
    for r in range(rounds):
        assert np.array_equal(both[0][r], alone[0][r]), r
    assert np.array_equal(both[1], alone[1])
    assert np.array_equal(both[2], alone[2])


def wait_done(lib, s, limit_s=60.0):
    t0 = time.time()
    while not lib.sjk_hip_seq_state_poll(C.byref(s)):
        assert time.time() - t0 < limit_s, "asynchronous state transfer did not finish"
        time.sleep(0.001)


def test_async_state_save_and_restore_while_decoding(lib, dev):
    cfg = config(lib)
    rows_a, rows_b = Rows(dev, 3400, seed=21), Rows(dev, 3400, seed=22)
    pool = new_pool(lib, cfg, blocks=160)
    a, b = new_seq(lib, cfg, pool), new_seq(lib, cfg, pool)
    c = d = None
    before, after = dev.alloc(rows_a.nq), dev.alloc(rows_a.nq)
    try:
        grow(lib, dev, a, rows_a, 2600, 10, None, True)
        grow(lib, dev, b, rows_b, 1500, 0, None, True)
        dev.sync()
        want = stream_bytes(lib, a)
        attend(lib, a, rows_a, before, None)
        n_a = int(a.n)
        # the save: begin, then keep decoding B and growing A while the host thread copies the snapshot out
        dst = np.zeros(want.nbytes, np.uint8)
        sjk.check(lib.sjk_hip_seq_state_write_begin(C.byref(a), dst.ctypes.data, dst.nbytes), "state_write_begin")
        assert lib.sjk_hip_seq_state_write_begin(C.byref(a), dst.ctypes.data, dst.nbytes) == sjk.ERR_PENDING
        w = C.c_size_t(0)
        assert lib.sj_kvarn_seq_state_write(C.byref(a), dst.ctypes.data, dst.nbytes, C.byref(w)) == sjk.ERR_PENDING
        for r in range(20):
            step(lib, b, rows_b, b.n, W, None, True)
            attend(lib, b, rows_b, after, None)
            step(lib, a, rows_a, a.n, W, None, True)
        wait_done(lib, a)
        sjk.check(lib.sjk_hip_seq_state_finish(C.byref(a), C.byref(w)), "state_finish")
        assert w.value == want.nbytes and a.n == n_a + 20 * W
        assert np.array_equal(dst, want)
        # the restore into a fresh sequence while B decodes
        c = new_seq(lib, cfg, pool)
        sjk.check(lib.sjk_hip_seq_state_read_begin(C.byref(c), dst.ctypes.data, dst.nbytes), "state_read_begin")
        for r in range(10):
            step(lib, b, rows_b, b.n, W, None, True)
            attend(lib, b, rows_b, after, None)
        wait_done(lib, c)
        sjk.check(lib.sjk_hip_seq_state_finish(C.byref(c), None), "state_finish")
        assert c.n == n_a and c.pol.B == int(np.frombuffer(want[96:100].tobytes(), np.uint32)[0])
        assert np.array_equal(stream_bytes(lib, c), want)
        attend(lib, c, rows_a, after, None)
        dev.sync()
        assert np.array_equal(dev.get(before, rows_a.nq, np.uint32), dev.get(after, rows_a.nq, np.uint32))
        # a damaged stream: the header passes at _begin, the checksum fails at _finish, the target is untouched
        d = new_seq(lib, cfg, pool)
        grow(lib, dev, d, rows_b, 700, 0, None, True)
        dev.sync()
        keep = stream_bytes(lib, d)
        bad = dst.copy()
        bad[200 + bad.nbytes // 2] ^= 1
        sjk.check(lib.sjk_hip_seq_state_read_begin(C.byref(d), bad.ctypes.data, bad.nbytes), "state_read_begin")
        assert lib.sjk_hip_seq_state_finish(C.byref(d), None) == sjk.ERR_CORRUPT
        assert np.array_equal(stream_bytes(lib, d), keep)
    finally:
        for s in (a, b, c, d):
            if s is not None:
                lib.sj_kvarn_seq_free(C.byref(s))
        lib.sj_kvarn_pool_free(C.byref(pool))


@pytest.mark.parametrize("Dw,staging", [(64, 1), (192, 1), (384, 0), (384, 1), (640, 0)])
def test_stage_rows_of_any_width(oracle, lib, dev, Dw, staging):
    """sjk_hip_stage and the drop-in sj_kvarn_stage_row at widths outside the row kernel's (128, 256, 512): fp16
    staging converts every value, tq6_0 the D / 128 whole blocks of each row (sj_kvarn.h:1221-1271)."""
    rng = np.random.default_rng(Dw)
    n = 9
    x = (rng.standard_normal((n, Dw)) * rng.lognormal(0, 2, (n, 1))).astype(np.float32)
    x[0, :3] = [np.inf, -0.0, 65520.0]
    rb = oracle.stage_row_bytes(staging, Dw)
    want = np.zeros((n, rb), np.uint8)
    for r in range(n):
        oracle.stage_row(staging, cabi.ptr(x[r], cabi.f32p), want[r].ctypes.data, Dw)
    dx, dy = dev.put(x), dev.alloc(n * rb)
    sjk.check(lib.sjk_hip_stage(staging, dx, dy, Dw, rb, n, None), "sjk_hip_stage")
    assert np.array_equal(dev.get(dy, n * rb, np.uint8).reshape(n, rb), want)
    # rows further apart than their staged size
    pitch = rb + 6
    dz = dev.alloc(n * pitch)
    sjk.check(lib.sjk_hip_stage(staging, dx, dz, Dw, pitch, n, None), "sjk_hip_stage pitch")
    got = dev.get(dz, n * pitch, np.uint8).reshape(n, pitch)[:, :rb]
    assert np.array_equal(got, want)
    one = np.zeros(rb, np.uint8)
    lib.sj_kvarn_stage_row(staging, cabi.ptr(x[1], sjk.f32p), one.ctypes.data, Dw)
    assert np.array_equal(one, want[1])
