"""The error contract of the sequence API on the product (libsjk.so, caches in HBM), ported from the reference's
tests/test_state.c with its shapes (D = 128, 2 KV heads, 2 layers, sink 128, tail 256 / 512):

  * the state-read rejection table (tests/test_state.c:270-348): every mismatch, damage and truncation of a stream
    is refused with the reference's status code, and the target sequence (which already holds 900 positions) is
    byte-for-byte what it was; a pool without enough free blocks refuses the stream and keeps its blocks;
  * a full pool refuses the seal and leaves the sequence as it was (tests/test_state.c:409-420);
  * truncate + re-prefill equals a fresh build (tests/test_state.c:129-189): for 12 cuts (past the end, in the tail,
    at / around B, on and inside group boundaries, in the sink, at 0) the resume point, B and n are the
    reference's, kept records are unchanged, dropped ones are zero, and after re-prefilling an edited suffix and
    an idle flush the stream payload and the attention outputs equal those of a sequence built fresh.

Everything except the checks runs through the product's sj_kvarn_* calls on the device; the conditions are forced
from the host.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import cabi

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

from test_gpu_layer import dump, st_grow, st_rows  # noqa: E402
from test_oracle_state import NL, mkcfg  # noqa: E402

pytestmark = pytest.mark.gpu
SINK, G, H, D = 128, 128, 2, 128
FNV0 = 1469598103934665603
NO = 0xFFFFFFFF


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


def cfg_of(oracle, bk, bv, body, **kw):
    c = sjk.Config.from_buffer_copy(bytes(mkcfg(oracle, bk, bv, body)))
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def new_seq(lib, cfg, n_layers=NL, pool=None):
    s = sjk.Seq()
    rc = lib.sj_kvarn_seq_init(C.byref(s), C.byref(cfg), n_layers, C.byref(pool) if pool is not None else None)
    return s, rc


def refix_checksum(x):
    h = FNV0
    for b in x[:-8].tobytes():
        h ^= b
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    x[-8:] = np.frombuffer(h.to_bytes(8, "little"), np.uint8)


def refix_fast(oracle, x):
    h = oracle.fnv1a(x.ctypes.data, x.nbytes - 8, FNV0)
    x[-8:] = np.frombuffer(int(h).to_bytes(8, "little"), np.uint8)


def test_state_read_rejection_table(oracle, lib):
    c = cfg_of(oracle, 3, 3, 1)
    a, rc = new_seq(lib, c)
    assert rc == 0
    try:
        assert st_grow(lib, a, 31, NO, 0, 0, 1300, 2) == 0
        s = dump(lib, a)
        info = sjk.StateInfo()
        assert lib.sj_kvarn_state_peek(s.ctypes.data, s.nbytes, C.byref(info)) == 0
        assert (info.n, info.B, info.n_layers, info.total_bytes, info.cfg.bits_k, info.cfg.body) == \
            (1300, a.pol.B, NL, s.nbytes, 3, 1)
    finally:
        lib.sj_kvarn_seq_free(C.byref(a))

    n_checked = [0]

    def expect(cfg, n_layers, stream, size, want, what):
        t, rc = new_seq(lib, cfg, n_layers)
        assert rc == 0, what
        try:
            assert st_grow(lib, t, 5, NO, 0, 0, 900, 1) == 0       # the target holds a sequence: it must survive
            before = dump(lib, t)
            got = lib.sj_kvarn_seq_state_read(C.byref(t), stream.ctypes.data, size)
            assert got == want, "%s: rc %d, want %d" % (what, got, want)
            assert np.array_equal(dump(lib, t), before), "%s: the failed restore changed the target" % what
            n_checked[0] += 1
        finally:
            lib.sj_kvarn_seq_free(C.byref(t))

    n = s.nbytes
    expect(cfg_of(oracle, 3, 3, 1, head_dim=256), NL, s, n, -120, "head_dim")
    expect(cfg_of(oracle, 3, 3, 1, n_head_kv=1), NL, s, n, -121, "n_head_kv")
    expect(cfg_of(oracle, 3, 3, 1, sink=192), NL, s, n, -123, "sink length")
    expect(cfg_of(oracle, 3, 3, 1, sink_type=1), NL, s, n, -123, "sink type")
    expect(cfg_of(oracle, 3, 3, 1, bits_v=2), NL, s, n, -124, "bits 3/2 vs 3/3")
    expect(cfg_of(oracle, 4, 4, 2), NL, s, n, -124, "bits 4/4 vs 3/3")
    expect(cfg_of(oracle, 3, 3, 0), NL, s, n, -125, "scalar vs trellis")
    expect(cfg_of(oracle, 3, 3, 1, iters=8), NL, s, n, -126, "iters")
    expect(cfg_of(oracle, 3, 3, 1, staging=1), NL, s, n, -127, "staging")
    expect(cfg_of(oracle, 3, 3, 1, tail=384), NL, s, n, -128, "tail")
    expect(cfg_of(oracle, 3, 3, 1, tail_max=1024), NL, s, n, -128, "tail_max")
    expect(cfg_of(oracle, 3, 3, 1, tail_max=0), NL, s, n, -128, "fixed vs adaptive tail")
    expect(cfg_of(oracle, 3, 3, 1, flush_chunk=2), NL, s, n, -128, "flush_chunk")
    expect(c, NL + 1, s, n, -131, "n_layers")
    expect(cfg_of(oracle, 3, 3, 1, n_ctx=1024), NL, s, n, -109, "context too small")
    # the reference's group mismatch needs a group-64 target; the device kernels are built for G = 128, so such a
    # layer is refused at creation (SJK_ERR_UNSUPPORTED) instead
    g64, rc = new_seq(lib, cfg_of(oracle, 4, 4, 0, group=64))
    assert rc == -141
    lib.sj_kvarn_seq_free(C.byref(g64))
    # header fields the config cannot express: rewritten, checksum fixed
    for off, val, want, what in ((72, 2, -129, "rotation id"), (76, 64, -129, "rotation size"),
                                 (80, None, -130, "codebook"), (12, 2, -106, "record format version")):
        x = s.copy()
        x[off] = (x[off] ^ 1) if val is None else val
        refix_fast(oracle, x)
        expect(c, NL, x, n, want, what)
    x = s.copy(); x[8] = 2; expect(c, NL, x, n, -105, "state version")                      # noqa: E702
    x = s.copy(); x[0] = ord("X"); expect(c, NL, x, n, -104, "magic")                        # noqa: E702
    x = s.copy(); x[n // 2] ^= 0x10; expect(c, NL, x, n, -107, "payload bit flip")           # noqa: E702
    x = s.copy(); x[n - 1] ^= 1; expect(c, NL, x, n, -107, "checksum")                       # noqa: E702
    x = s.copy(); x[96] = (int(x[96]) + 1) & 255; refix_fast(oracle, x)                      # noqa: E702
    expect(c, NL, x, n, -107, "B off a group boundary")
    x = s.copy(); x[92] = (int(x[92]) + 1) & 255; refix_fast(oracle, x)                      # noqa: E702
    expect(c, NL, x, n, -107, "n vs payload length")
    expect(c, NL, s, n - 1, -103, "one byte short")
    expect(c, NL, s, 100, -103, "header only")
    expect(c, NL, s, 4, -103, "4 bytes")
    # a pool without enough free blocks: refused, the pooled target keeps its (empty) state and the pool its blocks
    pool = sjk.Pool()
    assert lib.sj_kvarn_pool_init(C.byref(pool), C.byref(c), NL, 4) == 0
    q, rc = new_seq(lib, c, NL, pool)
    assert rc == 0
    assert lib.sj_kvarn_seq_state_read(C.byref(q), s.ctypes.data, n) == -110
    assert q.n == 0 and pool.n_free == 4
    lib.sj_kvarn_seq_free(C.byref(q))
    lib.sj_kvarn_pool_free(C.byref(pool))
    assert n_checked[0] == 28
    # the checksum helper agrees with the reference's (tests/test_state.c:252-257)
    y = s.copy(); y[40] ^= 4; z = y.copy(); refix_checksum(y); refix_fast(oracle, z)        # noqa: E702
    assert np.array_equal(y, z)


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 3, 1)], ids=["4/4", "3/3t"])
def test_full_pool_refuses_the_seal(oracle, lib, bk, bv, body):
    """tests/test_state.c:409-420: a pool of 2 blocks fills at the second group; the third seal is refused with
    POOL_FULL and the sequence keeps B = S + 2G with no seal pending."""
    c = cfg_of(oracle, bk, bv, body)
    pool = sjk.Pool()
    assert lib.sj_kvarn_pool_init(C.byref(pool), C.byref(c), NL, 2) == 0
    q, rc = new_seq(lib, c, NL, pool)
    assert rc == 0
    try:
        assert st_grow(lib, q, 51, NO, 0, 0, 1400, 1) == -110
        assert q.pol.B == SINK + 2 * G and q.pol.B_pending == q.pol.B
        assert pool.n_free == 0
    finally:
        lib.sj_kvarn_seq_free(C.byref(q))
        assert pool.n_free == 2
        lib.sj_kvarn_pool_free(C.byref(pool))


def records(lib, seq, il, n_groups):
    """device bytes of the records of groups [0, n_groups) of layer il, [g][h] order"""
    d = sjk.Device()
    L = seq.layers[il]
    out = []
    for g in range(n_groups):
        for h in range(H):
            p = lib.sj_kvarn_layer_record(C.byref(L), g, h)
            out.append(d.get(C.c_void_p(p), L.lay.bytes, np.uint8))
    return out


def attention(lib, seq):
    """outputs of sj_kvarn_seq_attend_row for 5 query positions per layer and head (tests/test_state.c:97-117)"""
    n = seq.n
    qp = [n - 1, n // 2, seq.pol.B - 1 if seq.pol.B > 0 else 0, seq.pol.B, 3]
    out = []
    o = np.zeros(D, np.float32)
    for il in range(NL):
        for h in range(H):
            for p0 in qp:
                p = p0 if p0 < n else n - 1
                q = st_rows(777, 0, p, (il * H + h + 1) * D, 0)[(il * H + h) * D:]
                lib.sj_kvarn_seq_attend_row(C.byref(seq), il, cabi.ptr(np.ascontiguousarray(q), cabi.f32p), h, p,
                                            0.0883883476, cabi.ptr(o, cabi.f32p))
                out.append(o.copy())
    return np.array(out)


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 3, 1)], ids=["4/4", "3/3t"])
def test_truncate_and_reprefill_equal_a_fresh_build(oracle, lib, bk, bv, body):
    c = cfg_of(oracle, bk, bv, body)
    N, M = 1500, 1760
    ref, rc = new_seq(lib, c)
    assert rc == 0
    try:
        assert st_grow(lib, ref, 11, NO, 0, 0, N, 1) == 0
        B0 = ref.pol.B
        assert B0 > SINK + 3 * G
        ref_recs = records(lib, ref, 1, (B0 - SINK) // G)
        cuts = [N + 50, N - 1, B0 + 7, B0, B0 - 1, B0 - G, B0 - G - 5, SINK + G + 1, SINK + 1, SINK, SINK - 10, 0]
        for cut in cuts:
            want_r = cut if (cut >= B0 or cut <= SINK) else SINK + G * ((cut - SINK) // G)
            want_B = B0 if cut >= B0 else (want_r if want_r > SINK else SINK)
            edit = min(cut, N)
            a, rc = new_seq(lib, c)
            f, rc2 = new_seq(lib, c)
            assert rc == 0 and rc2 == 0
            try:
                assert st_grow(lib, a, 11, NO, 0, 0, N, 1) == 0
                r = lib.sj_kvarn_seq_truncate(C.byref(a), cut)
                assert r == want_r and r <= cut and cut - r <= G - 1, (cut, r)
                assert a.pol.B == want_B and a.n == min(r, N), (cut, a.pol.B, a.n)
                recs = records(lib, a, 1, (B0 - SINK) // G)
                kept = (a.pol.B - SINK) // G
                for i, (x, y) in enumerate(zip(recs, ref_recs)):
                    if i // H < kept:
                        assert np.array_equal(x, y), "cut %d: kept record %d changed" % (cut, i // H)
                    else:
                        assert not x.any(), "cut %d: dropped record %d not zeroed" % (cut, i // H)
                # re-prefill the edited suffix with another ubatch pattern; a fresh build of the same rows
                assert st_grow(lib, a, 11, edit, 1, a.n, M, 3) == 0
                assert st_grow(lib, f, 11, edit, 1, 0, M, 2) == 0
                assert lib.sj_kvarn_seq_idle(C.byref(a), 0) == 0 and lib.sj_kvarn_seq_idle(C.byref(f), 0) == 0
                assert a.pol.B == f.pol.B and a.n == f.n, cut
                sa, sf = dump(lib, a), dump(lib, f)
                assert sa.nbytes == sf.nbytes and np.array_equal(sa[128:-8], sf[128:-8]), "cut %d: payload differs" % cut
                assert np.array_equal(attention(lib, a).view(np.uint32), attention(lib, f).view(np.uint32)), cut
            finally:
                lib.sj_kvarn_seq_free(C.byref(a))
                lib.sj_kvarn_seq_free(C.byref(f))
    finally:
        lib.sj_kvarn_seq_free(C.byref(ref))
