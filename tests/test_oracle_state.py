"""Oracle sequence / pool / state stream against the reference's golden stream hashes.

tests/golden/expected_state.txt holds FNV-1a 64 of the state stream of the reference test's 1500-position
build (tests/test_state.c:192-243 with N = 1500, seed 23, ubatch pattern 4) for five configs
(tests/test_state.c:432-438). The stream layout, the policy schedule, the pool and every record byte feed
these hashes.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

import cabi

GOLD = os.path.join(os.path.dirname(__file__), "golden", "expected_state.txt")
FNV0 = 1469598103934665603
NL, H, D = 2, 2, 128


def mkcfg(api, bk, bv, body, staging=0, sink_type=0, flush=0):
    c = api.config_default(D, H, 2304, 64)
    c.bits_k, c.bits_v, c.body = bk, bv, body
    c.sink, c.tail, c.tail_max = 128, 256, 512
    c.staging, c.sink_type, c.flush_chunk = staging, sink_type, flush
    return c


CONFIGS = {
    "4/4": dict(bk=4, bv=4, body=0),
    "3/3": dict(bk=3, bv=3, body=0),
    "3/3t": dict(bk=3, bv=3, body=1, flush=1),
    "3/2t": dict(bk=3, bv=2, body=1),
    "4/4f": dict(bk=4, bv=4, body=0, staging=1, sink_type=1, flush=1),
}


def golden():
    out = {}
    for line in open(GOLD):
        m = re.match(r"state (\S+) v1 hash=([0-9a-f]+)", line)
        if m:
            out[m.group(1)] = int(m.group(2), 16)
    return out


def dump(api, seq):
    n = api.seq_state_size(C.byref(seq))
    buf = np.zeros(n, np.uint8)
    w = C.c_size_t(0)
    rc = api.seq_state_write(C.byref(seq), buf.ctypes.data, n, C.byref(w))
    assert rc == 0 and w.value == n
    return buf


def test_golden_complete():
    assert set(golden()) == set(CONFIGS)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_state_stream_golden(oracle, name):
    cfg = mkcfg(oracle, **CONFIGS[name])
    seq = cabi.Seq()
    assert oracle.seq_init(C.byref(seq), C.byref(cfg), NL, None) == 0
    try:
        assert oracle.st_grow(C.byref(seq), 23, 0xFFFFFFFF, 0, 0, 1500, 4) == 0
        s = dump(oracle, seq)
        assert oracle.fnv1a(s.ctypes.data, s.nbytes, FNV0) == golden()[name]
        # the stream parses, and write -> read -> write is byte-identical (test_state.c:216-220)
        info = cabi.StateInfo()
        assert oracle.state_peek(s.ctypes.data, s.nbytes, C.byref(info)) == 0
        assert info.n == 1500 and info.total_bytes == s.nbytes and info.n_layers == NL
        other = cabi.Seq()
        cfg2 = mkcfg(oracle, **CONFIGS[name])
        cfg2.n_ubatch, cfg2.n_ctx = 512, 3304
        assert oracle.seq_init(C.byref(other), C.byref(cfg2), NL, None) == 0
        assert oracle.seq_state_read(C.byref(other), s.ctypes.data, s.nbytes) == 0
        assert np.array_equal(dump(oracle, other), s)
        oracle.seq_free(C.byref(other))
    finally:
        oracle.seq_free(C.byref(seq))


def test_state_rejections_leave_target_unchanged(oracle):
    """A sample of the reference's rejection table (tests/test_state.c:273-348)."""
    cfg = mkcfg(oracle, 3, 3, 1)
    a = cabi.Seq()
    assert oracle.seq_init(C.byref(a), C.byref(cfg), NL, None) == 0
    oracle.st_grow(C.byref(a), 31, 0xFFFFFFFF, 0, 0, 1300, 2)
    s = dump(oracle, a)

    def expect(cfg_m, nl, stream, want):
        t = cabi.Seq()
        assert oracle.seq_init(C.byref(t), C.byref(cfg_m), nl, None) == 0
        oracle.st_grow(C.byref(t), 5, 0xFFFFFFFF, 0, 0, 900, 1)
        before = dump(oracle, t)
        rc = oracle.seq_state_read(C.byref(t), stream.ctypes.data, stream.nbytes)
        after = dump(oracle, t)
        oracle.seq_free(C.byref(t))
        assert rc == want
        assert np.array_equal(before, after)

    m = mkcfg(oracle, 3, 3, 1); m.head_dim = 256; expect(m, NL, s, -120)
    m = mkcfg(oracle, 3, 3, 1); m.n_head_kv = 1; expect(m, NL, s, -121)
    m = mkcfg(oracle, 3, 3, 1); m.bits_v = 2; expect(m, NL, s, -124)
    m = mkcfg(oracle, 3, 3, 1); m.iters = 8; expect(m, NL, s, -126)
    m = mkcfg(oracle, 3, 3, 1); m.tail = 384; expect(m, NL, s, -128)
    m = mkcfg(oracle, 3, 3, 1); m.n_ctx = 1024; expect(m, NL, s, -109)
    expect(cfg, NL + 1, s, -131)
    x = s.copy(); x[0] = ord("X"); expect(cfg, NL, x, -104)
    x = s.copy(); x[len(x) // 2] ^= 0x10; expect(cfg, NL, x, -107)
    expect(cfg, NL, s[:-1].copy(), -103)
    oracle.seq_free(C.byref(a))


def test_pool_matches_alone(oracle):
    """Two sequences sharing a paged pool give the same streams as alone (tests/test_state.c:377-422)."""
    cfg = mkcfg(oracle, 4, 4, 0)
    pool = cabi.Pool()
    assert oracle.pool_init(C.byref(pool), C.byref(cfg), NL, 30) == 0
    pa, pb, la, lb = cabi.Seq(), cabi.Seq(), cabi.Seq(), cabi.Seq()
    oracle.seq_init(C.byref(pa), C.byref(cfg), NL, C.byref(pool))
    oracle.seq_init(C.byref(pb), C.byref(cfg), NL, C.byref(pool))
    oracle.seq_init(C.byref(la), C.byref(cfg), NL, None)
    oracle.seq_init(C.byref(lb), C.byref(cfg), NL, None)
    for p in range(0, 1400, 200):
        oracle.st_grow(C.byref(pa), 51, 0xFFFFFFFF, 0, p, p + 200, 1)
        oracle.st_grow(C.byref(la), 51, 0xFFFFFFFF, 0, p, p + 200, 1)
        oracle.st_grow(C.byref(pb), 52, 0xFFFFFFFF, 0, p, p + 200, 3)
        oracle.st_grow(C.byref(lb), 52, 0xFFFFFFFF, 0, p, p + 200, 3)
    r1 = oracle.seq_truncate(C.byref(pa), 900)
    r2 = oracle.seq_truncate(C.byref(la), 900)
    assert r1 == r2
    oracle.st_grow(C.byref(pb), 52, 0xFFFFFFFF, 0, 1400, 1900, 3)
    oracle.st_grow(C.byref(lb), 52, 0xFFFFFFFF, 0, 1400, 1900, 3)
    oracle.st_grow(C.byref(pa), 51, 900, 3, r1, 1700, 2)
    oracle.st_grow(C.byref(la), 51, 900, 3, r2, 1700, 2)
    jumps = sum(pb.blocks[g] != pb.blocks[g - 1] + 1 for g in range(1, (pb.pol.B - 128) // 128))
    assert jumps > 0
    assert np.array_equal(dump(oracle, pa), dump(oracle, la))
    assert np.array_equal(dump(oracle, pb), dump(oracle, lb))
    for s in (pa, pb, la, lb):
        oracle.seq_free(C.byref(s))
    assert pool.n_free == pool.n_blocks
    oracle.pool_free(C.byref(pool))
