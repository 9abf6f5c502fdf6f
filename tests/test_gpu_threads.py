"""Thread and stream safety of the device path (reference contract: per-sequence objects, no global mutable
state, callers serialise the use of one object, sj_kvarn.h:72-74). Two sequences are attended at the same time
from two host threads, each on a stream of its own (default priority), many calls in a row; every output must
equal, bit for bit, the output of the same call made alone. The calls keep their partial results in their own
sequence's workspace, so nothing is shared between the threads."""
import ctypes as C
import sys
import threading

import numpy as np
import pytest

import cabi
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 3, 1)], ids=["4/4s", "3/3t"])
def test_two_sequences_two_threads_two_streams(lib, bk, bv, body):
    D, H, n_head, n_q = 256, 4, 16, 4
    dev = sjk.Device()
    cfg = lib.sj_kvarn_config_default(D, H, 16384, 512)
    cfg.bits_k, cfg.bits_v, cfg.body = bk, bv, body
    pool = sjk.Pool()
    sjk.check(lib.sj_kvarn_pool_init(C.byref(pool), C.byref(cfg), 2, 2 * 130), "pool_init")
    seqs = [sjk.Seq(), sjk.Seq()]
    try:
        for s in seqs:
            sjk.check(lib.sj_kvarn_seq_init(C.byref(s), C.byref(cfg), 2, C.byref(pool)), "seq_init")
        # two different contexts (lengths, rows), built on the null stream
        for k, (s, n) in enumerate(zip(seqs, (9000, 11500))):
            for p0 in range(0, n, 512):
                m = min(512, n - p0)
                sjk.check(lib.sj_kvarn_seq_begin_ubatch(C.byref(s), p0, m), "begin_ubatch")
                K, V = inputs.kv_rows(m, H, D, seed=100 * k + p0)
                dK, dV = dev.put(K), dev.put(V)
                for il in range(2):
                    sjk.check(lib.sjk_hip_seq_store(C.byref(s), il, p0, m, dK, dV, 1, None), "seq_store")
                dev.sync()
                dev.free(dK)
                dev.free(dV)
        assert seqs[0].pol.B > 128 and seqs[1].pol.B > 128
        qs = [np.random.default_rng(k).standard_normal((n_q, n_head, D)).astype(np.float32) for k in range(2)]
        dq = [dev.put(q) for q in qs]
        n_calls = 60
        outs = [[dev.alloc(qs[k].nbytes) for _ in range(n_calls)] for k in range(2)]
        # alone: one call per sequence and layer, synchronised
        alone = []
        for k, s in enumerate(seqs):
            ref = dev.alloc(qs[k].nbytes)
            sjk.check(lib.sjk_hip_seq_attend(C.byref(s), 1, s.n - n_q, n_q, n_head, dq[k], 0.0625, ref, None), "attend")
            dev.sync()
            alone.append(dev.get(ref, qs[k].nbytes, np.uint32))
        streams = [dev.stream(), dev.stream()]
        errors = []
        start = threading.Barrier(2)

        def run(k):
            try:
                s = seqs[k]
                start.wait()
                for i in range(n_calls):
                    rc = lib.sjk_hip_seq_attend(C.byref(s), 1, s.n - n_q, n_q, n_head, dq[k], 0.0625, outs[k][i],
                                                streams[k])
                    if rc:
                        errors.append((k, i, rc))
                        return
                dev.hip.hipStreamSynchronize(streams[k])
            except Exception as e:  # noqa: BLE001
                errors.append((k, repr(e)))

        ths = [threading.Thread(target=run, args=(k,)) for k in range(2)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        assert not errors, errors
        for k in range(2):
            for i in range(n_calls):
                got = dev.get(outs[k][i], qs[k].nbytes, np.uint32)
                assert np.array_equal(got, alone[k]), (k, i)
        for st in streams:
            dev.hip.hipStreamDestroy(st)
    finally:
        for s in seqs:
            lib.sj_kvarn_seq_free(C.byref(s))
        lib.sj_kvarn_pool_free(C.byref(pool))
        dev.free_all()
