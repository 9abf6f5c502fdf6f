"""Device-resident layer cache: append (tq6_0 staging ring + fp16 sink, fused Hadamard), commit (seal
straight out of the ring), region-resolved rows and decode attention, against the CPU oracle; and the
sequence / pool / state API of libsjk.so against the reference's golden state-stream hashes
(tests/golden/expected_state.txt, the reference's tests/test_state.c build).

Bars: ring, sink and record bytes and resolved rows bit-exact; attention within max-abs 1e-3 and
rel 1e-3 of the oracle's fp32 loop (BASELINE north star tolerance).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import cabi
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

from test_oracle_state import CONFIGS, NL, golden, mkcfg  # noqa: E402

pytestmark = pytest.mark.gpu
FNV0 = 1469598103934665603
ATOL = RTOL = 1e-3


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.fixture(scope="module")
def dev():
    d = sjk.Device()
    yield d
    d.free_all()


def host_bytes(ptr, n):
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint8)), shape=(n,)).copy()


def make_pair(oracle, lib, D, H, bk, bv, body, tail, tail_max, n_ctx, n_ubatch=64, staging=0, sink_type=0):
    ocfg = oracle.config_default(D, H, n_ctx, n_ubatch)
    ocfg.bits_k, ocfg.bits_v, ocfg.body, ocfg.tail, ocfg.tail_max = bk, bv, body, tail, tail_max
    ocfg.staging, ocfg.sink_type = staging, sink_type
    OL = cabi.Layer()
    assert oracle.layer_init(C.byref(OL), C.byref(ocfg)) == 0
    pcfg = sjk.Config.from_buffer_copy(bytes(ocfg))
    PL = sjk.Layer()
    sjk.check(lib.sj_kvarn_layer_init(C.byref(PL), C.byref(pcfg)), "sj_kvarn_layer_init")
    return OL, PL


def oracle_store(oracle, OL, K, V, pos0):
    """engine order: rotate every head, then store (sj_kvarn.h:754-759, 1475-1492)"""
    n, H, D = K.shape
    for i in range(n):
        kr, vr = np.ascontiguousarray(K[i]).copy(), np.ascontiguousarray(V[i]).copy()
        oracle.rotate_heads(cabi.ptr(kr, cabi.f32p), H, D)
        oracle.rotate_heads(cabi.ptr(vr, cabi.f32p), H, D)
        oracle.layer_store(C.byref(OL), pos0 + i, cabi.ptr(kr, cabi.f32p), cabi.ptr(vr, cabi.f32p))


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 2, 1)], ids=["4/4s", "3/2t"])
def test_append_commit_rows_attention(oracle, lib, dev, bk, bv, body):
    D, H, S, G = 256, 4, 128, 128
    tail, tail_max = 256, 512
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, tail, tail_max, n_ctx=4096)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        n_pos = S + 5 * G + 37                      # sink + 5 groups + a ragged tail (ring cap 768)
        K, V = inputs.kv_rows(n_pos, H, D, seed=11 + bk)
        oracle_store(oracle, OL, K, V, 0)
        dK, dV = dev.put(K), dev.put(V)
        # two appends: a prefill chunk across the sink boundary, then the rest (fused rotation)
        cut = S + 50
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, cut, dK, dV, 1, None), "layer_store")
        off = cut * H * D * 4
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), cut, n_pos - cut, C.c_void_p(dK.value + off),
                                          C.c_void_p(dV.value + off), 1, None), "layer_store")
        dev.sync()
        sink_b = S * H * D * 4
        ring_b = OL.cap * H * 2 * OL.stage_bytes
        assert np.array_equal(dev.get(C.c_void_p(view.sink), sink_b, np.uint8), host_bytes(OL.sink, sink_b))
        assert np.array_equal(dev.get(C.c_void_p(view.ring), ring_b, np.uint8), host_bytes(OL.ring, ring_b))
        # commit 4 groups straight out of the ring in one launch
        B = S + 4 * G
        oracle.layer_seal(C.byref(OL), S, B)
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, B, 16, None), "commit")
        dev.sync()
        body_b = 4 * H * OL.lay.bytes
        got_body = dev.get(C.c_void_p(view.body), body_b, np.uint8)
        assert np.array_equal(got_body, host_bytes(OL.body, body_b))
        # resolved rows: sink, body and tail positions, bit-exact
        N = n_pos
        dk, dv = dev.alloc(N * D * 4), dev.alloc(N * D * 4)
        a, b = np.zeros(D, np.float32), np.zeros(D, np.float32)
        for h in (0, 3):
            sjk.check(lib.sjk_hip_kv_rows(C.byref(view), B, 0, N, h, dk, dv, None), "kv_rows")
            rk = dev.get(dk, N * D * 4, np.float32).reshape(N, D)
            rv = dev.get(dv, N * D * 4, np.float32).reshape(N, D)
            for p in (0, 127, 128, 300, B - 1, B, N - 1):
                oracle.layer_kv_row(C.byref(OL), B, p, h, cabi.ptr(a, cabi.f32p), cabi.ptr(b, cabi.f32p))
                assert np.array_equal(rk[p].view(np.uint32), a.view(np.uint32)), (h, p)
                assert np.array_equal(rv[p].view(np.uint32), b.view(np.uint32)), (h, p)
        # decode attention: width 4, 16 query heads (GQA 4:1), causal rows at the end of the context
        n_q, n_head = 4, 16
        q = np.random.default_rng(5).standard_normal((n_q, n_head, D)).astype(np.float32)
        qpos0 = N - n_q
        scale = 1.0 / 16.0
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, qpos0, n_q, n_head, dq, scale, do, None), "attend")
        got = dev.get(do, q.nbytes, np.float32).reshape(n_q, n_head, D)
        want = np.zeros_like(got)
        for iq in range(n_q):
            for hq in range(n_head):
                qq = np.ascontiguousarray(q[iq, hq])
                oracle.layer_attend_row(C.byref(OL), B, N, cabi.ptr(qq, cabi.f32p), hq // (n_head // H), qpos0 + iq,
                                        scale, cabi.ptr(want[iq, hq], cabi.f32p))
        err = np.abs(got - want)
        assert np.all(err <= ATOL + RTOL * np.abs(want)), "max abs err %g" % err.max()
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("staging", [0, 1], ids=["tq6", "f16"])
@pytest.mark.parametrize("rotate", [0, 1], ids=["plain", "rotated"])
@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 2, 1), (3, 3, 1)], ids=["4/4s", "3/2t", "3/3t"])
def test_commit_nonfinite_rows_from_the_ring(oracle, lib, dev, bk, bv, body, rotate, staging):
    """Rows holding +-inf and NaNs of both signs appended through the device store (with and without the fused
    rotation, tq6_0 and fp16 staging), then sealed out of the ring by one commit: sink, ring and records against
    the oracle's layer_store + layer_seal (sj_kvarn.h:1475-1514). Codes and every non-NaN value byte for byte;
    NaN values and NaN scales NaN on both sides (their sign is left to operand order where NaNs of both signs meet,
    which a rotation of a row with an infinity already makes happen)."""
    D, H, S, G = 256, 2, 128, 128
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, tail=256, tail_max=512, n_ctx=2048, staging=staging)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        n_pos = S + 3 * G + 21
        K, V = inputs.kv_rows(n_pos, H, D, seed=31 + bk + staging)
        rng = np.random.default_rng(rotate + 2 * staging)
        specials = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFA00055], np.uint32)
        for X in (K, V):
            m = rng.random(X.shape) < 0.002
            X.view(np.uint32)[m] = rng.choice(specials, int(m.sum()))
        K[S + 5, 1, :] = np.inf                     # a whole row of one head
        V[S + G + 7, 0, :] = -np.inf
        K[S + 2 * G:S + 3 * G, 0, 3] = np.inf       # one channel over a whole group
        for i in range(n_pos):
            kr, vr = K[i].copy(), V[i].copy()
            if rotate:
                oracle.rotate_heads(cabi.ptr(kr, cabi.f32p), H, D)
                oracle.rotate_heads(cabi.ptr(vr, cabi.f32p), H, D)
            oracle.layer_store(C.byref(OL), i, cabi.ptr(kr, cabi.f32p), cabi.ptr(vr, cabi.f32p))
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, rotate, None), "layer_store")
        dev.sync()
        sink_b = S * H * D * 4
        got = dev.get(C.c_void_p(view.sink), sink_b, np.uint16)
        assert inputs.halves_equal_nan_unsigned(got, host_bytes(OL.sink, sink_b).view(np.uint16)).all()
        ring_b = OL.cap * H * 2 * OL.stage_bytes
        got = dev.get(C.c_void_p(view.ring), ring_b, np.uint8)
        want = host_bytes(OL.ring, ring_b)
        if staging == 0:
            assert inputs.tq6_mismatch(got, want).size == 0
        else:
            assert inputs.halves_equal_nan_unsigned(got.view(np.uint16), want.view(np.uint16)).all()
        if not rotate:
            assert np.array_equal(got, want), "without rotation the stored rows keep their own NaN signs"
        B = S + 3 * G
        oracle.layer_seal(C.byref(OL), S, B)
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, B, 16, None), "commit")
        dev.sync()
        nrec = 3 * H
        got = dev.get(C.c_void_p(view.body), nrec * OL.lay.bytes, np.uint8).reshape(nrec, -1)
        want = host_bytes(OL.body, nrec * OL.lay.bytes).reshape(nrec, -1)
        for r in range(nrec):
            bad = inputs.record_mismatch(OL.lay, got[r], want[r])
            assert bad.size == 0, (r, bad[:8])
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


ATT_CASES = [
    # staging, sink_type, n_pos, n_q, n_head, commit groups, qpos offset from the end
    (0, 0, 128 + 9 * 128 + 301, 4, 16, 9, 0),       # tq6_0 tail, fp16 sink, width 4 GQA 4:1
    (1, 0, 128 + 4 * 128 + 77, 2, 8, 4, 0),         # fp16 staging tail
    (0, 1, 128 + 3 * 128 + 200, 1, 4, 3, 0),        # sink stored in the staging type, width 1
    (0, 0, 128 + 9 * 128 + 301, 4, 16, 9, 500),     # causal rows inside the body: later records masked
]


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 3, 1), (4, 2, 0)], ids=["4/4s", "3/3t", "4/2s"])
@pytest.mark.parametrize("D", [256, 128], ids=["d256", "d128"])
@pytest.mark.parametrize("staging,sink_type,n_pos,n_q,n_head,ngr,back", ATT_CASES,
                         ids=["tq6-f16sink", "f16-staging", "inherit-sink", "rows-in-body"])
def test_attention_regions_vs_oracle(oracle, lib, dev, staging, sink_type, n_pos, n_q, n_head, ngr, back, D, bk, bv,
                                     body):
    """Every region combination (sink type, staging type, causal rows inside the body) on the 4/4, trellis and
    other scalar-body kernels; the sealed records byte-equal to the oracle's first."""
    H, S, G = 4, 128, 128
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=4096, n_ubatch=512, staging=staging,
                       sink_type=sink_type)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        K, V = inputs.kv_rows(n_pos, H, D, seed=31 + staging + 2 * sink_type)
        oracle_store(oracle, OL, K, V, 0)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, 1, None), "layer_store")
        B = S + ngr * G
        oracle.layer_seal(C.byref(OL), S, B)
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, B, 16, None), "commit")
        dev.sync()
        # the records sealed out of this ring (tq6_0 or fp16 staging rows), byte for byte
        body_b = ngr * H * OL.lay.bytes
        assert np.array_equal(dev.get(C.c_void_p(view.body), body_b, np.uint8), host_bytes(OL.body, body_b))
        q = np.random.default_rng(8).standard_normal((n_q, n_head, D)).astype(np.float32) * np.float32(2.0)
        qpos0 = n_pos - n_q - back
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        sjk.check(lib.sjk_hip_attend(C.byref(view), B, n_pos, qpos0, n_q, n_head, dq, 0.0625, do, None), "attend")
        got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
        want = np.zeros_like(got)
        for iq in range(n_q):
            for hq in range(n_head):
                qq = np.ascontiguousarray(q[iq, hq])
                oracle.layer_attend_row(C.byref(OL), B, n_pos, cabi.ptr(qq, cabi.f32p), hq // (n_head // H), qpos0 + iq,
                                        0.0625, cabi.ptr(want[iq, hq], cabi.f32p))
        err = np.abs(got - want)
        assert np.all(err <= ATOL + RTOL * np.abs(want)), "max abs err %g" % err.max()
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("D", [256, 128], ids=["d256", "d128"])
def test_attention_long_context_many_workgroups(oracle, lib, dev, D):
    """Enough sealed records that every KV head spreads over many workgroups (partials + combine)."""
    H, S, G = 4, 128, 128
    n_ctx = 128 + 300 * 128 + 1024
    OL, PL = make_pair(oracle, lib, D, H, 4, 4, 0, 256, 512, n_ctx=n_ctx, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        B = S + 300 * G
        n_pos = B + 300
        # store and seal on the device in windows that fit the ring (store and seal bytes are checked by the
        # tests above), then give the oracle layer the same sink, ring and record bytes
        stored = 0
        Bcur = S
        while stored < n_pos:
            n = min(512, n_pos - stored)
            K, V = inputs.kv_rows(n, H, D, seed=1000 + stored)
            dK, dV = dev.put(K), dev.put(V)
            sjk.check(lib.sjk_hip_layer_store(C.byref(view), stored, n, dK, dV, 1, None), "layer_store")
            stored += n
            target = min(B, S + (max(stored - 256, S) - S) // G * G)
            if target > Bcur:
                sjk.check(lib.sjk_hip_commit(C.byref(view), 1, Bcur, target, 16, None), "commit")
                Bcur = target
        assert Bcur == B
        dev.sync()
        for name, nb in (("sink", S * H * D * 4), ("ring", OL.cap * H * 2 * OL.stage_bytes),
                         ("body", 300 * H * OL.lay.bytes)):
            b = dev.get(C.c_void_p(getattr(view, name)), nb, np.uint8)
            C.memmove(getattr(OL, name), b.ctypes.data, nb)
        n_q, n_head = 4, 16
        q = np.random.default_rng(9).standard_normal((n_q, n_head, D)).astype(np.float32)
        qpos0 = n_pos - n_q
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        sjk.check(lib.sjk_hip_attend(C.byref(view), B, n_pos, qpos0, n_q, n_head, dq, 0.0625, do, None), "attend")
        got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
        for iq, hq in ((0, 0), (3, 15), (1, 6), (2, 9)):
            want = np.zeros(D, np.float32)
            qq = np.ascontiguousarray(q[iq, hq])
            oracle.layer_attend_row(C.byref(OL), B, n_pos, cabi.ptr(qq, cabi.f32p), hq // 4, qpos0 + iq, 0.0625,
                                    cabi.ptr(want, cabi.f32p))
            err = np.abs(got[iq, hq] - want)
            assert np.all(err <= ATOL + RTOL * np.abs(want)), "row (%d,%d) max abs err %g" % (iq, hq, err.max())
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


def device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed, window=512):
    """Store n_pos positions and seal [S, B) on the device in ring-sized windows, then give the oracle
    layer the device's sink, ring and record bytes (store and seal bytes are checked bit-exact above)."""
    H, D, S, G = OL.cfg.n_head_kv, OL.cfg.head_dim, OL.cfg.sink, 128
    stored, Bcur = 0, S
    while stored < n_pos:
        n = min(window, n_pos - stored)
        K, V = inputs.kv_rows(n, H, D, seed=seed + stored)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), stored, n, dK, dV, 1, None), "layer_store")
        stored += n
        target = min(B, S + (max(stored - 256, S) - S) // G * G)
        if target > Bcur:
            sjk.check(lib.sjk_hip_commit(C.byref(view), 1, Bcur, target, 16, None), "commit")
            Bcur = target
    assert Bcur == B
    dev.sync()
    for name, nb in (("sink", S * H * D * 4), ("ring", OL.cap * H * 2 * OL.stage_bytes),
                     ("body", (B - S) // G * H * OL.lay.bytes)):
        if nb:
            b = dev.get(C.c_void_p(getattr(view, name)), nb, np.uint8)
            C.memmove(getattr(OL, name), b.ctypes.data, nb)


def attend_check(oracle, lib, dev, OL, view, B, n_pos, qpos0, q, scale, rows=None):
    n_q, n_head, D = q.shape
    H = OL.cfg.n_head_kv
    dq, do = dev.put(q), dev.alloc(q.nbytes)
    sjk.check(lib.sjk_hip_attend(C.byref(view), B, n_pos, qpos0, n_q, n_head, dq, scale, do, None), "attend")
    got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
    rows = rows or [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
    worst = 0.0
    for iq, hq in rows:
        want = np.zeros(D, np.float32)
        qq = np.ascontiguousarray(q[iq, hq])
        oracle.layer_attend_row(C.byref(OL), B, n_pos, cabi.ptr(qq, cabi.f32p), hq // (n_head // H), qpos0 + iq,
                                scale, cabi.ptr(want, cabi.f32p))
        err = np.abs(got[iq, hq] - want)
        assert np.all(err <= ATOL + RTOL * np.abs(want)), "row (%d,%d) max abs err %g" % (iq, hq, err.max())
        worst = max(worst, float((err / (ATOL + RTOL * np.abs(want))).max()))
    return worst


TR_BODIES = [(3, 3), (3, 2), (2, 2)]


@pytest.mark.parametrize("D", [256, 128], ids=["d256", "d128"])
@pytest.mark.parametrize("bk,bv", TR_BODIES, ids=["3/3t", "3/2t", "2/2t"])
@pytest.mark.parametrize("ngr,back", [(9, 0), (9, 500), (1, 0)], ids=["tail", "rows-in-body", "one-record"])
def test_attention_trellis_vs_oracle(oracle, lib, dev, bk, bv, ngr, back, D):
    """Trellis records on the matrix-core path: every channel's window decode (zero history at the
    stream start, pairs straddling words), the fp16 sink and tq6_0 tail, causal masking in the body."""
    H, S, G = 4, 128, 128
    n_pos = S + ngr * G + 301
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, 1, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        B = S + ngr * G
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=300 + 10 * bk + bv)
        n_q, n_head = 4, 16
        q = np.random.default_rng(12).standard_normal((n_q, n_head, D)).astype(np.float32) * np.float32(2.0)
        attend_check(oracle, lib, dev, OL, view, B, n_pos, n_pos - n_q - back, q, 0.0625)
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("D", [256, 128], ids=["d256", "d128"])
def test_attention_trellis_long_context(oracle, lib, dev, D):
    """3/3 trellis body over 300 groups: many record workgroups per KV head, partials + combine."""
    H, S, G = 4, 128, 128
    B = S + 300 * G
    n_pos = B + 300
    OL, PL = make_pair(oracle, lib, D, H, 3, 3, 1, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=2000)
        q = np.random.default_rng(13).standard_normal((4, 16, D)).astype(np.float32)
        attend_check(oracle, lib, dev, OL, view, B, n_pos, n_pos - 4, q, 0.0625,
                     rows=[(0, 0), (3, 15), (1, 6), (2, 9)])
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


BATCH_CASES = [(4, 4, 0, 256), (3, 3, 1, 256), (4, 4, 0, 128), (4, 2, 0, 256), (3, 3, 1, 128), (2, 3, 0, 128)]


@pytest.mark.parametrize("bk,bv,body,D", BATCH_CASES,
                         ids=["4/4s", "3/3t", "d128-4/4s", "4/2s", "d128-3/3t", "d128-2/3s"])
def test_store_and_attend_batch(oracle, lib, dev, bk, bv, body, D):
    """sjk_hip_store_batch writes the bytes of one sjk_hip_layer_store per job; sjk_hip_attend_batch
    (one launch for jobs of different context lengths) agrees with sjk_hip_attend per job and with the
    oracle."""
    H, S, G = 4, 128, 128
    ctx = [(S + 3 * G + 300, 3), (S + 9 * G + 301, 9), (S + 40, 0)]         # (positions, sealed groups)
    pairs = [make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=n + 64, n_ubatch=512) for n, _ in ctx]
    views = [lib.sjk_layer_view(C.byref(PL)) for _, PL in pairs]
    try:
        for k, ((n_pos, ngr), (OL, PL)) in enumerate(zip(ctx, pairs)):
            device_context(oracle, lib, dev, OL, PL, views[k], n_pos, S + ngr * G, seed=500 + 31 * k)
        # one more ubatch of 4 positions, stored by one batched launch into all three layers
        K, V = inputs.kv_rows(4, H, D, seed=77)
        dK, dV = dev.put(K), dev.put(V)
        jobs = (sjk.StoreJob * 3)()
        for k, (n_pos, _) in enumerate(ctx):
            jobs[k].v, jobs[k].pos0, jobs[k].d_k, jobs[k].d_v = views[k], n_pos, dK.value, dV.value
        sjk.check(lib.sjk_hip_store_batch(jobs, 3, 4, 1, None), "store_batch")
        for k, ((n_pos, ngr), (OL, PL)) in enumerate(zip(ctx, pairs)):
            oracle_store(oracle, OL, K, V, n_pos)
            dev.sync()
            nb = OL.cap * H * 2 * OL.stage_bytes
            assert np.array_equal(dev.get(C.c_void_p(views[k].ring), nb, np.uint8), host_bytes(OL.ring, nb)), k
            nb = S * H * D * 4
            assert np.array_equal(dev.get(C.c_void_p(views[k].sink), nb, np.uint8), host_bytes(OL.sink, nb)), k
        n_q, n_head = 4, 16
        q = np.random.default_rng(14).standard_normal((3, n_q, n_head, D)).astype(np.float32)
        dqs = [dev.put(q[k]) for k in range(3)]
        outs = [dev.alloc(q[k].nbytes) for k in range(3)]
        single = [dev.alloc(q[k].nbytes) for k in range(3)]
        ajobs = (sjk.AttendJob * 3)()
        for k, (n_pos, ngr) in enumerate(ctx):
            N = n_pos + 4
            ajobs[k].v, ajobs[k].B, ajobs[k].N, ajobs[k].qpos0 = views[k], S + ngr * G, N, N - n_q
            ajobs[k].d_q, ajobs[k].d_out = dqs[k].value, outs[k].value
            sjk.check(lib.sjk_hip_attend(C.byref(views[k]), S + ngr * G, N, N - n_q, n_q, n_head, dqs[k], 0.0625,
                                         single[k], None), "attend")
        sjk.check(lib.sjk_hip_attend_batch(ajobs, 3, n_q, n_head, 0.0625, None), "attend_batch")
        for k, (n_pos, ngr) in enumerate(ctx):
            got = dev.get(outs[k], q[k].nbytes, np.float32).reshape(q[k].shape)
            one = dev.get(single[k], q[k].nbytes, np.float32).reshape(q[k].shape)
            assert np.allclose(got, one, rtol=1e-5, atol=1e-6), k
            N = n_pos + 4
            worst = 0.0
            for iq in range(n_q):
                for hq in (0, 5, 10, 15):
                    want = np.zeros(D, np.float32)
                    qq = np.ascontiguousarray(q[k, iq, hq])
                    OL = pairs[k][0]
                    oracle.layer_attend_row(C.byref(OL), S + ngr * G, N, cabi.ptr(qq, cabi.f32p), hq // 4, N - n_q + iq,
                                            0.0625, cabi.ptr(want, cabi.f32p))
                    err = np.abs(got[iq, hq] - want)
                    assert np.all(err <= ATOL + RTOL * np.abs(want)), (k, iq, hq, err.max())
    finally:
        for OL, PL in pairs:
            oracle.layer_free(C.byref(OL))
            lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 3, 1)], ids=["4/4s", "3/3t"])
@pytest.mark.parametrize("n_q", [5, 12], ids=["20rows", "48rows"])
def test_attend_batch_wide_rows(oracle, lib, dev, bk, bv, body, n_q):
    """sjk_hip_attend_batch of three calls (different contexts) with more than 16 query rows per KV head: their
    16-row tiles are the jobs (6 of them at 20 rows, 9 at 48 rows: more than one launch), each call's result
    agrees with its own sjk_hip_attend and with the oracle, for every row."""
    H, S, G, D = 4, 128, 128, 256
    ctx = [(S + 3 * G + 300, 3), (S + 9 * G + 301, 9), (S + 40, 0)]         # (positions, sealed groups)
    pairs = [make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=n + 64, n_ubatch=512) for n, _ in ctx]
    views = [lib.sjk_layer_view(C.byref(PL)) for _, PL in pairs]
    try:
        for k, ((n_pos, ngr), (OL, PL)) in enumerate(zip(ctx, pairs)):
            device_context(oracle, lib, dev, OL, PL, views[k], n_pos, S + ngr * G, seed=600 + 31 * k)
        n_head = 16
        q = np.random.default_rng(19 + n_q).standard_normal((3, n_q, n_head, D)).astype(np.float32)
        dqs = [dev.put(q[k]) for k in range(3)]
        outs = [dev.alloc(q[k].nbytes) for k in range(3)]
        single = [dev.alloc(q[k].nbytes) for k in range(3)]
        ajobs = (sjk.AttendJob * 3)()
        for k, (n_pos, ngr) in enumerate(ctx):
            ajobs[k].v, ajobs[k].B, ajobs[k].N, ajobs[k].qpos0 = views[k], S + ngr * G, n_pos, n_pos - n_q
            ajobs[k].d_q, ajobs[k].d_out = dqs[k].value, outs[k].value
            sjk.check(lib.sjk_hip_attend(C.byref(views[k]), S + ngr * G, n_pos, n_pos - n_q, n_q, n_head, dqs[k],
                                         0.0625, single[k], None), "attend")
        sjk.check(lib.sjk_hip_attend_batch(ajobs, 3, n_q, n_head, 0.0625, None), "attend_batch")
        for k, (n_pos, ngr) in enumerate(ctx):
            got = dev.get(outs[k], q[k].nbytes, np.float32).reshape(q[k].shape)
            one = dev.get(single[k], q[k].nbytes, np.float32).reshape(q[k].shape)
            assert np.allclose(got, one, rtol=1e-5, atol=1e-6), k
            OL = pairs[k][0]
            for iq in range(n_q):
                for hq in range(n_head):
                    want = np.zeros(D, np.float32)
                    qq = np.ascontiguousarray(q[k, iq, hq])
                    oracle.layer_attend_row(C.byref(OL), S + ngr * G, n_pos, cabi.ptr(qq, cabi.f32p), hq // 4,
                                            n_pos - n_q + iq, 0.0625, cabi.ptr(want, cabi.f32p))
                    err = np.abs(got[iq, hq] - want)
                    assert np.all(err <= ATOL + RTOL * np.abs(want)), (k, iq, hq, err.max())
    finally:
        for OL, PL in pairs:
            oracle.layer_free(C.byref(OL))
            lib.sj_kvarn_layer_free(C.byref(PL))


def test_attend_batch_mixed_layouts(oracle, lib, dev):
    """sjk_hip_attend_batch with jobs of different layouts (4/4, 3/3 trellis, 4/2 scalar, and 4/4 at D = 128 with
    8 KV heads: no two share a launch) runs one call per job; each result equals that job's sjk_hip_attend bit for
    bit and agrees with the oracle."""
    S, G = 128, 128
    specs = [(256, 4, 4, 4, 0), (256, 4, 3, 3, 1), (256, 4, 4, 2, 0), (128, 8, 4, 4, 0)]
    n_q, n_head_per_kv = 4, 4
    pairs = [make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=S + 5 * G + 200, n_ubatch=512)
             for D, H, bk, bv, body in specs]
    views = [lib.sjk_layer_view(C.byref(PL)) for _, PL in pairs]
    try:
        n_pos, B = S + 4 * G + 300, S + 4 * G
        for k, ((OL, PL), spec) in enumerate(zip(pairs, specs)):
            device_context(oracle, lib, dev, OL, PL, views[k], n_pos, B, seed=900 + 17 * k)
        # all jobs share n_q and n_head: 32 query heads (GQA 8:1 on 4 KV heads, 4:1 on 8)
        n_head = 32
        qs = [np.random.default_rng(40 + k).standard_normal((n_q, n_head, spec[0])).astype(np.float32)
              for k, spec in enumerate(specs)]
        dqs = [dev.put(q) for q in qs]
        outs = [dev.alloc(q.nbytes) for q in qs]
        single = [dev.alloc(q.nbytes) for q in qs]
        jobs = (sjk.AttendJob * len(specs))()
        for k in range(len(specs)):
            jobs[k].v, jobs[k].B, jobs[k].N, jobs[k].qpos0 = views[k], B, n_pos, n_pos - n_q
            jobs[k].d_q, jobs[k].d_out = dqs[k].value, outs[k].value
            sjk.check(lib.sjk_hip_attend(C.byref(views[k]), B, n_pos, n_pos - n_q, n_q, n_head, dqs[k], 0.0625,
                                         single[k], None), "attend")
        sjk.check(lib.sjk_hip_attend_batch(jobs, len(specs), n_q, n_head, 0.0625, None), "attend_batch")
        for k, (D, H, bk, bv, body) in enumerate(specs):
            got = dev.get(outs[k], qs[k].nbytes, np.float32).reshape(qs[k].shape)
            one = dev.get(single[k], qs[k].nbytes, np.float32).reshape(qs[k].shape)
            assert np.array_equal(got, one), k
            OL = pairs[k][0]
            for iq, hq in ((0, 0), (n_q - 1, n_head - 1), (2, 13)):
                want = np.zeros(D, np.float32)
                qq = np.ascontiguousarray(qs[k][iq, hq])
                oracle.layer_attend_row(C.byref(OL), B, n_pos, cabi.ptr(qq, cabi.f32p), hq // (n_head // H),
                                        n_pos - n_q + iq, 0.0625, cabi.ptr(want, cabi.f32p))
                assert np.all(np.abs(got[iq, hq] - want) <= ATOL + RTOL * np.abs(want)), (k, iq, hq)
    finally:
        for OL, PL in pairs:
            oracle.layer_free(C.byref(OL))
            lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("bk,bv,body,D", [(4, 4, 0, 256), (3, 3, 1, 256), (4, 4, 0, 128), (3, 3, 0, 256), (3, 2, 1, 128)],
                         ids=["4/4s", "3/3t", "d128-4/4s", "3/3s", "d128-3/2t"])
def test_attention_vs_float64(oracle, lib, dev, bk, bv, body, D):
    """Decode attention against float64 attention over the oracle's decoded rows (KV head 0, 20K context):
    within a quarter of the parity tolerance, independent of the rounding of the reference's fp32 loop
    (whose own distance to float64 is printed for comparison)."""
    H, S, G = 4, 128, 128
    n_groups = 150
    B = S + n_groups * G
    n_pos = B + 900
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 1024, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=4000 + bk)
        n_q, n_head = 4, 16
        q = np.random.default_rng(15).standard_normal((n_q, n_head, D)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        sjk.check(lib.sjk_hip_attend(C.byref(view), B, n_pos, n_pos - n_q, n_q, n_head, dq, 0.0625, do, None), "attend")
        got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
        K = np.zeros((n_pos, D), np.float32)
        V = np.zeros((n_pos, D), np.float32)
        for p in range(n_pos):
            oracle.layer_kv_row(C.byref(OL), B, p, 0, cabi.ptr(K[p], cabi.f32p), cabi.ptr(V[p], cabi.f32p))
        K64, V64 = K.astype(np.float64), V.astype(np.float64)
        worst_gpu = worst_ref = 0.0
        for iq in range(n_q):
            for hq in range(4):                           # the query heads of KV head 0
                qp = n_pos - n_q + iq
                sc = (K64[:qp + 1] @ q[iq, hq].astype(np.float64)) * 0.0625
                pw = np.exp(sc - sc.max())
                ref = (pw @ V64[:qp + 1]) / pw.sum()
                tol = ATOL + RTOL * np.abs(ref)
                worst_gpu = max(worst_gpu, float(np.max(np.abs(got[iq, hq] - ref) / tol)))
                want = np.zeros(D, np.float32)
                qq = np.ascontiguousarray(q[iq, hq])
                oracle.layer_attend_row(C.byref(OL), B, n_pos, cabi.ptr(qq, cabi.f32p), 0, qp, 0.0625,
                                        cabi.ptr(want, cabi.f32p))
                worst_ref = max(worst_ref, float(np.max(np.abs(want - ref) / tol)))
        print("error / tolerance vs float64: device %.4f, reference loop %.4f" % (worst_gpu, worst_ref))
        assert worst_gpu <= 0.25, worst_gpu
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


EDGE_BODIES = [(4, 4, 0), (3, 3, 1), (4, 2, 0)]


@pytest.mark.parametrize("bk,bv,body", EDGE_BODIES, ids=["4/4s", "3/3t", "4/2s"])
@pytest.mark.parametrize("D", [256, 128], ids=["d256", "d128"])
def test_attention_edge_cases(oracle, lib, dev, D, bk, bv, body):
    """Only the sink (N <= S), a query row at position 0, and positions past qpos are masked: the row path of
    the 4/4, trellis and other scalar-body kernels."""
    H, S = 4, 128
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=2048)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        n_pos = 100
        K, V = inputs.kv_rows(n_pos, H, D, seed=21)
        oracle_store(oracle, OL, K, V, 0)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, 1, None), "layer_store")
        n_q, n_head = 3, 8
        q = np.random.default_rng(6).standard_normal((n_q, n_head, D)).astype(np.float32)
        for qpos0 in (0, 40):
            dq, do = dev.put(q), dev.alloc(q.nbytes)
            sjk.check(lib.sjk_hip_attend(C.byref(view), S, n_pos, qpos0, n_q, n_head, dq, 0.0625, do, None), "attend")
            got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
            want = np.zeros_like(got)
            for iq in range(n_q):
                for hq in range(n_head):
                    qq = np.ascontiguousarray(q[iq, hq])
                    oracle.layer_attend_row(C.byref(OL), S, n_pos, cabi.ptr(qq, cabi.f32p), hq // (n_head // H),
                                            qpos0 + iq, 0.0625, cabi.ptr(want[iq, hq], cabi.f32p))
            assert np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


# ---- sequences, pool and state stream through the product API --------------------------------------

def _sm_mix(x):
    x = (x + np.uint64(0x9E3779B97F4A7C15)) & np.uint64(0xFFFFFFFFFFFFFFFF)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def st_rows(seed, variant, pos, n, side):
    """values of tests/test_state.c:40-45 for indices 0..n-1 of one position (vectorised)"""
    i = np.arange(n, dtype=np.uint64)
    key = (np.uint64(seed) << np.uint64(40)) ^ (np.uint64(variant) << np.uint64(36)) ^ \
          (np.uint64(pos) << np.uint64(16)) ^ (i << np.uint64(1)) ^ np.uint64(side)
    with np.errstate(over="ignore"):
        h = _sm_mix(key)
    g = (h & np.uint64(1023)).astype(np.int64) + ((h >> np.uint64(10)) & np.uint64(1023)).astype(np.int64) - 1024
    sc = np.where(i % np.uint64(41) == 0, 24, 1 + ((h >> np.uint64(20)) & np.uint64(3)).astype(np.int64))
    return ((g * sc).astype(np.float32) * np.float32(1.0 / 4096.0)).astype(np.float32)


def st_grow(lib, seq, seed, edit_from, edit_variant, frm, to, pattern):
    """tests/test_state.c:55-74 through the product's sequence API"""
    row = seq.n_layers * seq.cfg.n_head_kv * seq.cfg.head_dim
    pos, step = frm, 0
    while pos < to:
        n = 1 if pattern == 0 else (1 + (pattern * 7 + step * 13) % 64 if step % 5 == 4 else 1 + (step + pattern) % 4)
        n = min(n, to - pos)
        rc = lib.sj_kvarn_seq_begin_ubatch(C.byref(seq), pos, n)
        if rc:
            return rc
        for p in range(pos, pos + n):
            var = edit_variant if p >= edit_from else 0
            k, v = st_rows(seed, var, p, row, 0), st_rows(seed, var, p, row, 1)
            lib.sj_kvarn_seq_store(C.byref(seq), p, cabi.ptr(k, cabi.f32p), cabi.ptr(v, cabi.f32p))
        pos += n
        step += 1
    return 0


def dump(lib, seq):
    n = lib.sj_kvarn_seq_state_size(C.byref(seq))
    buf = np.zeros(n, np.uint8)
    w = C.c_size_t(0)
    sjk.check(lib.sj_kvarn_seq_state_write(C.byref(seq), buf.ctypes.data, n, C.byref(w)), "state_write")
    assert w.value == n
    return buf


def test_st_rows_matches_oracle_generator(oracle):
    row = 512
    got = st_rows(23, 3, 777, row, 1)
    want = np.array([oracle.st_val(23, 3, 777, i, 1) for i in range(row)], np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_state_stream_golden_on_device(oracle, lib, name):
    cfg = sjk.Config.from_buffer_copy(bytes(mkcfg(oracle, **CONFIGS[name])))
    seq = sjk.Seq()
    sjk.check(lib.sj_kvarn_seq_init(C.byref(seq), C.byref(cfg), NL, None), "seq_init")
    try:
        assert st_grow(lib, seq, 23, 0xFFFFFFFF, 0, 0, 1500, 4) == 0
        s = dump(lib, seq)
        assert oracle.fnv1a(s.ctypes.data, s.nbytes, FNV0) == golden()[name]
        other = sjk.Seq()
        cfg2 = sjk.Config.from_buffer_copy(bytes(cfg))
        cfg2.n_ubatch, cfg2.n_ctx = 512, 3304
        sjk.check(lib.sj_kvarn_seq_init(C.byref(other), C.byref(cfg2), NL, None), "seq_init")
        sjk.check(lib.sj_kvarn_seq_state_read(C.byref(other), s.ctypes.data, s.nbytes), "state_read")
        assert np.array_equal(dump(lib, other), s)
        lib.sj_kvarn_seq_free(C.byref(other))
    finally:
        lib.sj_kvarn_seq_free(C.byref(seq))


def test_pool_truncate_matches_alone_on_device(oracle, lib):
    """Pool vs alone, truncation and re-prefill (tests/test_state.c:377-422) on the device cache."""
    cfg = sjk.Config.from_buffer_copy(bytes(mkcfg(oracle, 4, 4, 0)))
    pool = sjk.Pool()
    sjk.check(lib.sj_kvarn_pool_init(C.byref(pool), C.byref(cfg), NL, 30), "pool_init")
    pa, pb, la, lb = sjk.Seq(), sjk.Seq(), sjk.Seq(), sjk.Seq()
    for s, pl in ((pa, C.byref(pool)), (pb, C.byref(pool)), (la, None), (lb, None)):
        sjk.check(lib.sj_kvarn_seq_init(C.byref(s), C.byref(cfg), NL, pl), "seq_init")
    for p in range(0, 1400, 200):
        st_grow(lib, pa, 51, 0xFFFFFFFF, 0, p, p + 200, 1)
        st_grow(lib, la, 51, 0xFFFFFFFF, 0, p, p + 200, 1)
        st_grow(lib, pb, 52, 0xFFFFFFFF, 0, p, p + 200, 3)
        st_grow(lib, lb, 52, 0xFFFFFFFF, 0, p, p + 200, 3)
    r1 = lib.sj_kvarn_seq_truncate(C.byref(pa), 900)
    r2 = lib.sj_kvarn_seq_truncate(C.byref(la), 900)
    assert r1 == r2
    st_grow(lib, pb, 52, 0xFFFFFFFF, 0, 1400, 1900, 3)
    st_grow(lib, lb, 52, 0xFFFFFFFF, 0, 1400, 1900, 3)
    st_grow(lib, pa, 51, 900, 3, r1, 1700, 2)
    st_grow(lib, la, 51, 900, 3, r2, 1700, 2)
    jumps = sum(pb.blocks[g] != pb.blocks[g - 1] + 1 for g in range(1, (pb.pol.B - 128) // 128))
    assert jumps > 0
    assert np.array_equal(dump(lib, pa), dump(lib, la))
    assert np.array_equal(dump(lib, pb), dump(lib, lb))
    for s in (pa, pb, la, lb):
        lib.sj_kvarn_seq_free(C.byref(s))
    assert pool.n_free == pool.n_blocks
    lib.sj_kvarn_pool_free(C.byref(pool))


@pytest.mark.gpu
def test_commit_dyn_graph_replay(oracle, lib, dev):
    """sjk_hip_commit_dyn captured once in a HIP graph and replayed for three commits whose ranges are
    only in the device descriptor (the fixed-size launch of the reference's seal_dyn,
    INTEGRATION_LLAMACPP.md:48-71): the records equal the oracle's sj_kvarn_layer_seal of the same ring
    rows, an empty range writes nothing, groups past a range stay untouched, and refused descriptors (negative
    entries, a range longer than the launch, misaligned ones) write nothing."""
    D, H, S, G = 256, 4, 128, 128
    OL, PL = make_pair(oracle, lib, D, H, 4, 4, 0, 256, 768, n_ctx=4096)
    view = lib.sjk_layer_view(C.byref(PL))
    hip = dev.hip
    hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
    hip.hipGraphDestroy.argtypes = [C.c_void_p]
    stream = dev.stream()
    graph, gexec = C.c_void_p(), C.c_void_p()
    try:
        n_pos = S + 6 * G + 10
        K, V = inputs.kv_rows(n_pos, H, D, seed=29)
        oracle_store(oracle, OL, K, V, 0)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, 1, None), "layer_store")
        dev.sync()
        desc = np.zeros(16, np.int32)
        d_desc = dev.put(desc)
        dev._ck(hip.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")       # relaxed capture
        rc = lib.sjk_hip_commit_dyn(C.byref(view), 1, d_desc, 4, 16, stream)
        dev._ck(hip.hipStreamEndCapture(stream, C.byref(graph)), "hipStreamEndCapture")
        sjk.check(rc, "commit_dyn")
        dev._ck(hip.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
        rec = OL.lay.bytes * H
        body_b = 6 * rec

        def replay(b_old, b):
            desc[9], desc[2] = b_old, b                  # SJK_DESC_B_OLD, SJK_DESC_B
            dev._ck(hip.hipMemcpy(d_desc, desc.ctypes.data, desc.nbytes, 1), "hipMemcpy")
            dev._ck(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
            dev._ck(hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
            return dev.get(C.c_void_p(view.body), body_b, np.uint8)

        zero = np.zeros(body_b, np.uint8)
        got = replay(S, S + 2 * G)
        oracle.layer_seal(C.byref(OL), S, S + 2 * G)
        want = host_bytes(OL.body, body_b)
        assert np.array_equal(got[:2 * rec], want[:2 * rec])
        assert np.array_equal(got[2 * rec:], zero[2 * rec:])
        assert np.array_equal(replay(S + 2 * G, S + 2 * G), got)              # empty range: nothing written
        got = replay(S + 2 * G, S + 5 * G)
        oracle.layer_seal(C.byref(OL), S + 2 * G, S + 5 * G)
        want = host_bytes(OL.body, body_b)
        assert np.array_equal(got[:5 * rec], want[:5 * rec])
        assert np.array_equal(got[5 * rec:], zero[5 * rec:])
        # refused, nothing written: negative entries (aligned on S + k G as unsigned), a range of 5 groups in a
        # launch of 4, a misaligned one
        for b_old, b in ((-256, -128), (-128, S + 6 * G), (S + G, S + 6 * G), (S + 5 * G + 1, S + 6 * G)):
            assert np.array_equal(replay(b_old, b), got), (b_old, b)
        got = replay(S + 5 * G, S + 6 * G)
        oracle.layer_seal(C.byref(OL), S + 5 * G, S + 6 * G)
        assert np.array_equal(got, host_bytes(OL.body, body_b))
    finally:
        if gexec.value:
            hip.hipGraphExecDestroy(gexec)
        if graph.value:
            hip.hipGraphDestroy(graph)
        lib.sj_kvarn_layer_free(C.byref(PL))
        oracle.layer_free(C.byref(OL))


@pytest.mark.gpu
@pytest.mark.parametrize("D,bk,bv,body,n_q,n_head", [(256, 4, 4, 0, 4, 16), (256, 3, 3, 1, 4, 16), (256, 3, 2, 1, 4, 16),
                                                     (256, 2, 2, 1, 4, 16), (128, 4, 4, 0, 4, 16), (128, 4, 2, 0, 4, 16),
                                                     (256, 3, 2, 0, 4, 16), (128, 3, 3, 1, 4, 16),
                                                     (256, 4, 4, 0, 5, 16), (128, 4, 4, 0, 4, 32), (256, 4, 2, 0, 5, 16),
                                                     (128, 3, 3, 0, 8, 16), (256, 3, 3, 1, 5, 16), (128, 4, 4, 0, 40, 16),
                                                     (128, 2, 2, 1, 8, 16), (256, 3, 2, 0, 40, 16)],
                         ids=["4/4s", "3/3t", "3/2t", "2/2t", "d128-4/4s", "d128-4/2s", "3/2s", "d128-3/3t",
                              "4/4s-20rows", "d128-4/4s-32rows", "4/2s-20rows", "d128-3/3s-32rows", "3/3t-20rows",
                              "d128-4/4s-160rows", "d128-2/2t-32rows", "3/2s-160rows"])
def test_attend_dyn_graph_replay(oracle, lib, dev, D, bk, bv, body, n_q, n_head):
    """sjk_hip_attend_dyn captured once in a HIP graph and replayed over contexts that are only in the device
    descriptor (the region-aware flash_attn_ext of INTEGRATION_LLAMACPP.md:49), for the 4/4 scalar and the
    three trellis bodies, and for 20, 32 and 160 query rows per KV head (width 5 at GQA 4:1, width 4 at GQA 8:1,
    width 8 at GQA 4:1, 40-position prefills: the 16-row tiles are the jobs of one launch, split on the device by
    the eager call's own arithmetic, 8 tiles a launch, all in the one graph; one replay has tiles that see different
    numbers of records, so that their shares differ): every replay equals sjk_hip_attend on the same
    (B, N, qpos0) bit for bit, the first also the oracle's
    sj_kvarn_layer_attend rows; descriptors the view cannot hold give NaN rows and leave the next replay correct. (Trellis bodies: the oracle attends over the
    device's records, whose bytes other tests hold equal to the oracle's seal.)"""
    H, S, G = 4, 128, 128
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 768, n_ctx=4096)
    view = lib.sjk_layer_view(C.byref(PL))
    hip = dev.hip
    hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
    hip.hipGraphDestroy.argtypes = [C.c_void_p]
    stream = dev.stream()
    graph, gexec = C.c_void_p(), C.c_void_p()
    try:
        n_pos = S + 9 * G + 301
        B = S + 9 * G
        K, V = inputs.kv_rows(n_pos, H, D, seed=31)
        oracle_store(oracle, OL, K, V, 0)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, 1, None), "layer_store")
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, B, 16, None), "commit")
        dev.sync()
        if body == 0:
            oracle.layer_seal(C.byref(OL), S, B)
        else:
            nb = (B - S) // G * H * PL.lay.bytes
            body_b = dev.get(C.c_void_p(PL.body), nb, np.uint8)
            C.memmove(OL.body, body_b.ctypes.data, nb)
        scale = 0.0625
        q = np.random.default_rng(11).standard_normal((n_q, n_head, D)).astype(np.float32)
        dq, do, dref = dev.put(q), dev.alloc(q.nbytes), dev.alloc(q.nbytes)
        desc = np.zeros(16, np.int32)
        d_desc = dev.put(desc)

        def set_desc(b, n, qpos0):
            desc[2], desc[3], desc[4] = b, n, qpos0              # SJK_DESC_B, SJK_DESC_N, SJK_DESC_QPOS0
            dev._ck(hip.hipMemcpy(d_desc, desc.ctypes.data, desc.nbytes, 1), "hipMemcpy")

        def reference(b, n, qpos0):
            sjk.check(lib.sjk_hip_attend(C.byref(view), b, n, qpos0, n_q, n_head, dq, scale, dref, None), "attend")
            dev.sync()
            return dev.get(dref, q.nbytes, np.float32)

        # eager call first: it allocates the call's buffers outside the capture
        set_desc(B, n_pos, n_pos - n_q)
        sjk.check(lib.sjk_hip_attend_dyn(C.byref(view), d_desc, 4096, n_q, n_head, dq, scale, do, None), "attend_dyn")
        dev.sync()
        got = dev.get(do, q.nbytes, np.float32)
        assert np.array_equal(got.view(np.uint32), reference(B, n_pos, n_pos - n_q).view(np.uint32))
        want = np.zeros((n_q, n_head, D), np.float32)
        for iq in range(n_q):
            for hq in range(n_head):
                qq = np.ascontiguousarray(q[iq, hq])
                oracle.layer_attend_row(C.byref(OL), B, n_pos, cabi.ptr(qq, cabi.f32p), hq // (n_head // H),
                                        n_pos - n_q + iq, scale, cabi.ptr(want[iq, hq], cabi.f32p))
        err = np.abs(got.reshape(want.shape) - want)
        assert np.all(err <= ATOL + RTOL * np.abs(want)), "max abs err %g" % err.max()

        dev._ck(hip.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")       # relaxed capture
        rc = lib.sjk_hip_attend_dyn(C.byref(view), d_desc, 4096, n_q, n_head, dq, scale, do, stream)
        dev._ck(hip.hipStreamEndCapture(stream, C.byref(graph)), "hipStreamEndCapture")
        sjk.check(rc, "attend_dyn")
        dev._ck(hip.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")

        def replay(b, n, qpos0):
            set_desc(b, n, qpos0)
            dev._ck(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
            dev._ck(hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
            return dev.get(do, q.nbytes, np.float32)

        cases = [
            (B, n_pos, n_pos - n_q),              # the eager call's context
            (B, n_pos - 50, n_pos - 50 - n_q),    # shorter tail
            (B, n_pos, n_pos - 500),              # causal rows inside the body: later records masked
            (S + 8 * G, S + 8 * G + 200, S + 8 * G + 196),
            (B, n_pos, S + 7 * G - 4),            # tiles across a record's end: the last tile sees one more record
            (S, S + 100, S + 96),                 # sink and tail only
            (0, 60, 56),                          # sink rows only
            (B, n_pos, n_pos - n_q),
        ]
        for b, n, qp in cases:
            got = replay(b, n, qp)
            assert np.array_equal(got.view(np.uint32), reference(b, n, qp).view(np.uint32)), (b, n, qp)
        assert S + view.cap + 10 <= 4096
        for b, n, qp in [(B + 1, n_pos, n_pos - n_q),      # B inside a group
                         (B, 5000, 4996),                  # N past n_max
                         (B, B - 10, B - 10 - n_q),        # B past N
                         (S, S + view.cap + 10, S + view.cap + 6)]:   # tail longer than the ring
            assert np.all(np.isnan(replay(b, n, qp))), (b, n, qp)
        got = replay(B, n_pos, n_pos - n_q)
        assert np.array_equal(got.view(np.uint32), reference(B, n_pos, n_pos - n_q).view(np.uint32))
    finally:
        if gexec.value:
            hip.hipGraphExecDestroy(gexec)
        if graph.value:
            hip.hipGraphDestroy(graph)
        lib.sj_kvarn_layer_free(C.byref(PL))
        oracle.layer_free(C.byref(OL))


@pytest.mark.gpu
def test_layer_store_dyn_graph_replay(oracle, lib, dev):
    """sjk_hip_layer_store_dyn captured once in a HIP graph and replayed for decode steps of 4 positions whose
    first position is only in the device descriptor: the sink and ring bytes equal those that
    sjk_hip_layer_store writes for the same rows into a second layer; a negative position stores nothing."""
    D, H, S = 256, 4, 128
    OL, PL = make_pair(oracle, lib, D, H, 4, 4, 0, 256, 768, n_ctx=4096)
    OL2, PL2 = make_pair(oracle, lib, D, H, 4, 4, 0, 256, 768, n_ctx=4096)
    view, view2 = lib.sjk_layer_view(C.byref(PL)), lib.sjk_layer_view(C.byref(PL2))
    hip = dev.hip
    hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
    hip.hipGraphDestroy.argtypes = [C.c_void_p]
    stream = dev.stream()
    graph, gexec = C.c_void_p(), C.c_void_p()
    try:
        w = 4
        n_pos = S + view.cap + 40                       # the sink, the ring, and a wrap of the ring
        K, V = inputs.kv_rows(n_pos, H, D, seed=37)
        step_b = w * H * D * 4
        dK, dV = dev.alloc(step_b), dev.alloc(step_b)
        desc = np.zeros(16, np.int32)
        d_desc = dev.put(desc)
        dev._ck(hip.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")       # relaxed capture
        rc = lib.sjk_hip_layer_store_dyn(C.byref(view), d_desc, w, dK, dV, 1, stream)
        dev._ck(hip.hipStreamEndCapture(stream, C.byref(graph)), "hipStreamEndCapture")
        sjk.check(rc, "layer_store_dyn")
        dev._ck(hip.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
        sink_b = S * H * 4 * D
        ring_b = view.cap * H * 2 * view.stage_bytes

        def state(v):
            return (dev.get(C.c_void_p(v.sink), sink_b, np.uint8), dev.get(C.c_void_p(v.ring), ring_b, np.uint8))

        for p0 in range(0, n_pos - w + 1, w):
            kk, vv = np.ascontiguousarray(K[p0:p0 + w]), np.ascontiguousarray(V[p0:p0 + w])
            dev._ck(hip.hipMemcpy(dK, kk.ctypes.data, step_b, 1), "hipMemcpy")
            dev._ck(hip.hipMemcpy(dV, vv.ctypes.data, step_b, 1), "hipMemcpy")
            desc[4] = p0                                 # SJK_DESC_QPOS0
            dev._ck(hip.hipMemcpy(d_desc, desc.ctypes.data, desc.nbytes, 1), "hipMemcpy")
            dev._ck(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
            dev._ck(hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
            sjk.check(lib.sjk_hip_layer_store(C.byref(view2), p0, w, dK, dV, 1, None), "layer_store")
            dev.sync()
        got, want = state(view), state(view2)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
        assert np.any(got[1] != 0)
        desc[4] = -1                                     # a negative position: nothing stored
        dev._ck(hip.hipMemcpy(d_desc, desc.ctypes.data, desc.nbytes, 1), "hipMemcpy")
        dev._ck(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
        dev._ck(hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
        again = state(view)
        assert np.array_equal(again[0], got[0]) and np.array_equal(again[1], got[1])
    finally:
        if gexec.value:
            hip.hipGraphExecDestroy(gexec)
        if graph.value:
            hip.hipGraphDestroy(graph)
        lib.sj_kvarn_layer_free(C.byref(PL))
        lib.sj_kvarn_layer_free(C.byref(PL2))
        oracle.layer_free(C.byref(OL))
        oracle.layer_free(C.byref(OL2))
