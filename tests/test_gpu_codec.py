"""Parity of the HIP codec kernels with the reference, through the C ABI of libsjk.so.

Bit-exact bars: sealed record bytes, tq6_0 bytes and decoded rows. Checked against
  * the reference's own known-answer vectors (tests/golden/expected_vectors.txt: 20 seal configs at
    D = 128/256 and the tq6_0 vector), hashed with the reference's protocol (tests/test_vectors.c:20-70);
  * the CPU oracle on seeded inputs at the BASELINE shapes (H = 4, D = 256, config-2 distributions),
    byte for byte, for every body the reference's device test covers (tests/test_cuda.cu:16).
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import cabi
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

from test_oracle_vectors import SEAL, TQ6  # noqa: E402

pytestmark = pytest.mark.gpu
FNV0 = 1469598103934665603


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.fixture(scope="module")
def dev():
    d = sjk.Device()
    yield d
    d.free_all()


def play(lay):
    """oracle layout -> product ctypes layout (same ABI)"""
    return sjk.Layout.from_buffer_copy(bytes(lay))


def oracle_seal(oracle, lay, K, V, row_stride, iters=16):
    rec = np.zeros(lay.bytes, np.uint8)
    work = np.zeros(oracle.seal_workspace_bytes(C.byref(lay)), np.uint8)
    oracle.seal_group(C.byref(lay), cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p), row_stride, iters, cabi.ptr(rec),
                      work.ctypes.data_as(C.c_void_p))
    return rec


@pytest.mark.parametrize("D,bk,bv,body,nbytes,erec,edec", SEAL,
                         ids=["D%d-%d/%d-%s" % (s[0], s[1], s[2], "t" if s[3] else "s") for s in SEAL])
def test_seal_known_answer_vectors(oracle, lib, dev, D, bk, bv, body, nbytes, erec, edec):
    lay = oracle.layout(D, 128, bk, bv, body)
    K = np.zeros(D * 128, np.uint16)
    V = np.zeros(D * 128, np.uint16)
    oracle.vec_fill_group(D, 128, 1, cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p))
    dK, dV, dR = dev.put(K), dev.put(V), dev.alloc(lay.bytes)
    sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dK, dV, D, 1, 1, 16, dR, None), "sjk_hip_seal")
    rec = dev.get(dR, lay.bytes, np.uint8)
    assert oracle.fnv1a(rec.ctypes.data, rec.nbytes, FNV0) == erec
    dk, dv = dev.alloc(128 * D * 4), dev.alloc(128 * D * 4)
    sjk.check(lib.sjk_hip_decode(C.byref(play(lay)), dR, 1, dk, dv, None), "sjk_hip_decode")
    rk = dev.get(dk, 128 * D * 4, np.float32).reshape(128, D)
    rv = dev.get(dv, 128 * D * 4, np.float32).reshape(128, D)
    rows = np.stack([rk, rv], axis=1)            # t-major, K then V per token (test_vectors.c:40-47)
    assert oracle.fnv1a(rows.ctypes.data, rows.nbytes, FNV0) == edec


def say(*a):
    print(*a, flush=True)


KL_CONFIGS = [(4, 4, 0), (3, 3, 1), (3, 2, 1), (2, 2, 1), (3, 3, 0), (3, 2, 0), (2, 2, 0)]    # test_kl.c:36


def kl_expected():
    """(bits_k, bits_v, body) -> (mean KL, max KL, mean output error) printed by the reference's test_kl"""
    out = {}
    for line in open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "expected_kl.txt")):
        f = line.split()
        if len(f) == 6 and "/" in f[0]:
            bk, bv = (int(x) for x in f[0].split("/"))
            out[(bk, bv, 1 if f[1] == "trellis" else 0)] = (float(f[3]), float(f[4]), float(f[5]))
    return out


KL_EXPECTED = kl_expected()


def kl_queries(Kx_groups, n_q):
    """The reference KL check's queries (test_kl.c:71-88): per group, n_q times a key of the group (xorshift pick)
    plus noise (sum of four uniforms / 600 of its magnitude), scaled so that the exact logits have standard
    deviation 2.5; the xorshift64 state starts at 12345 and runs on over the groups (vector_inputs.h:8-18)."""
    M = (1 << 64) - 1
    st = [12345]

    def nxt():
        s = st[0]
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        st[0] = s
        return (s >> 11) & 0xFFFFFFFF

    out = []
    for Kx in Kx_groups:
        G, D = Kx.shape
        qs = np.zeros((n_q, D))
        for qi in range(n_q):
            src = nxt() % G
            noise = np.array([sum(int(nxt() & 1023) - 512 for _ in range(4)) for _ in range(D)], np.float64)
            q = Kx[src] + noise / 600.0 * np.abs(Kx[src])
            a = Kx @ q
            m1 = a.mean()
            m2 = (a * a).mean() - m1 * m1
            qs[qi] = q * (2.5 / np.sqrt(m2) if m2 > 0 else 1.0)
        out.append(qs)
    return out


def test_kl_sanity_like_the_reference(oracle, lib, dev):
    """The reference's KL sanity check (tests/test_kl.c) on the device's seal and decode: 8 synthetic groups
    (sjv_fill_group seeds 7..14, D = 256, G = 128), 64 peaked queries each, for the 7 bodies of test_kl.c: the
    mean KL divergence of the decoded attention from the exact one finite and below 10, the mean relative output
    error below 1, and KL ordered by K bits over the scalar bodies (4/4 < 3/3 < 2/2). The device's records and
    decoded rows are also the oracle's bit for bit, so these are the reference's own figures."""
    D, G, NG, NQ = 256, 128, 8, 64
    groups = []
    for i in range(NG):
        K = np.zeros(D * G, np.uint16)
        V = np.zeros(D * G, np.uint16)
        oracle.vec_fill_group(D, G, i + 7, cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p))
        groups.append((K, V))
    Kx = [K.view(np.float16).astype(np.float64).reshape(G, D) for K, _ in groups]
    Vx = [V.view(np.float16).astype(np.float64).reshape(G, D) for _, V in groups]
    queries = kl_queries(Kx, NQ)
    kl_mean = {}
    dk, dv = dev.alloc(G * D * 4), dev.alloc(G * D * 4)
    for bk, bv, body in KL_CONFIGS:
        lay = oracle.layout(D, G, bk, bv, body)
        dR = dev.alloc(lay.bytes)
        kls, errs = [], []
        for i, (K, V) in enumerate(groups):
            sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dev.put(K), dev.put(V), D, 1, 1, 16, dR, None), "sjk_hip_seal")
            rec = dev.get(dR, lay.bytes, np.uint8)
            assert np.array_equal(rec, oracle_seal(oracle, lay, K, V, D)), (bk, bv, body, i)
            sjk.check(lib.sjk_hip_decode(C.byref(play(lay)), dR, 1, dk, dv, None), "sjk_hip_decode")
            Kd = dev.get(dk, G * D * 4, np.float32).reshape(G, D)
            Vd = dev.get(dv, G * D * 4, np.float32).reshape(G, D)
            want = np.zeros(D, np.float32)
            for t in (0, 77, G - 1):
                oracle.decode_k_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(want, cabi.f32p))
                assert np.array_equal(Kd[t].view(np.uint32), want.view(np.uint32)), (bk, bv, body, i, t)
            Kd, Vd = Kd.astype(np.float64), Vd.astype(np.float64)
            for q in queries[i]:
                sx, sd = Kx[i] @ q, Kd @ q
                px = np.exp(sx - sx.max())
                pd = np.exp(sd - sd.max())
                px, pd = px / px.sum(), pd / pd.sum()
                nz = px > 0
                kls.append(float(np.sum(px[nz] * np.log(px[nz] / np.maximum(pd[nz], 1e-300)))))
                ox, od = px @ Vx[i], pd @ Vd
                errs.append(float(np.sqrt(np.sum((ox - od) ** 2) / max(np.sum(ox * ox), 1e-300))))
        kl_mean[(bk, bv, body)] = np.mean(kls)
        say("[kl] %d/%d %-7s mean KL %.3e  max KL %.3e  out rel err %.3e" % (bk, bv, "trellis" if body else "scalar",
                                                                          np.mean(kls), max(kls), np.mean(errs)))
        assert 0.0 <= np.mean(kls) < 10.0 and np.mean(errs) < 1.0, (bk, bv, body)
        # the reference's own run of this check (tests/golden/expected_kl.txt, 4 significant digits)
        ref = KL_EXPECTED[(bk, bv, body)]
        got = (np.mean(kls), max(kls), np.mean(errs))
        assert all(abs(g - r) <= 1e-3 * r for g, r in zip(got, ref)), (bk, bv, body, got, ref)
    assert kl_mean[(4, 4, 0)] < kl_mean[(3, 3, 0)] < kl_mean[(2, 2, 0)]


def test_tq6_known_answer_vector(oracle, lib, dev):
    rows, n, eenc, edec = TQ6[0]
    x = np.zeros(rows * n, np.float32)
    oracle.vec_fill_rows(rows, n, cabi.ptr(x, cabi.f32p))
    rb = (n // 128) * 98
    dx, dq, dy = dev.put(x), dev.alloc(rows * rb), dev.alloc(rows * n * 4)
    sjk.check(lib.sjk_hip_stage(0, dx, dq, n, rb, rows, None), "sjk_hip_stage")
    q = dev.get(dq, rows * rb, np.uint8)
    assert oracle.fnv1a(q.ctypes.data, q.nbytes, FNV0) == eenc
    sjk.check(lib.sjk_hip_unstage(0, dq, rb, dy, n, rows, None), "sjk_hip_unstage")
    y = dev.get(dy, rows * n * 4, np.float32)
    assert oracle.fnv1a(y.ctypes.data, y.nbytes, FNV0) == edec


BODIES = [(4, 4, 0), (3, 3, 1), (3, 2, 1), (2, 2, 1), (3, 3, 0), (4, 2, 0), (2, 2, 0)]


@pytest.mark.parametrize("bk,bv,body", BODIES, ids=["%d/%d%s" % (a, b, "t" if c else "s") for a, b, c in BODIES])
def test_seal_baseline_shape_vs_oracle(oracle, lib, dev, bk, bv, body):
    """H = 4, D = 256, config-2 distributions; 3 groups x 4 heads sealed in one launch from token-major
    fp16 rows [pos][H][D] (row_stride = H*D), every record compared byte for byte, then decoded."""
    H, D, G, NG = 4, 256, 128, 3
    lay = oracle.layout(D, G, bk, bv, body)
    K, V = inputs.kv_rows(NG * G, H, D, seed=100 + 10 * bk + bv + body)
    Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
    dK, dV, dR = dev.put(Kh), dev.put(Vh), dev.alloc(NG * H * lay.bytes)
    sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dK, dV, H * D, H, NG, 16, dR, None), "sjk_hip_seal")
    got = dev.get(dR, NG * H * lay.bytes, np.uint8).reshape(NG * H, lay.bytes)
    for r in range(NG * H):
        g, h = divmod(r, H)
        off = g * G * H * D + h * D
        want = oracle_seal(oracle, lay, Kh[off:], Vh[off:], H * D)
        bad = np.nonzero(got[r] != want)[0]
        assert bad.size == 0, "record %d differs at %d bytes, first at %d" % (r, bad.size, bad[0])
    # decoded rows of every record are bit-exact
    dk, dv = dev.alloc(NG * H * G * D * 4), dev.alloc(NG * H * G * D * 4)
    sjk.check(lib.sjk_hip_decode(C.byref(play(lay)), dR, NG * H, dk, dv, None), "sjk_hip_decode")
    rk = dev.get(dk, NG * H * G * D * 4, np.float32).reshape(NG * H, G, D)
    rv = dev.get(dv, NG * H * G * D * 4, np.float32).reshape(NG * H, G, D)
    row = np.zeros(D, np.float32)
    for r in (0, NG * H - 1):
        rec = np.ascontiguousarray(got[r])
        for t in range(0, G, 7):
            oracle.decode_k_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(row, cabi.f32p))
            assert np.array_equal(rk[r, t].view(np.uint32), row.view(np.uint32))
            oracle.decode_v_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(row, cabi.f32p))
            assert np.array_equal(rv[r, t].view(np.uint32), row.view(np.uint32))


def test_seal_iters_and_c1_shape(oracle, lib, dev):
    """Config 1 (D = 128, one head, 4/4, outlier channels 3 and 77) and non-default iteration counts."""
    K, V = inputs.kv_rows_c1(seed=0)
    Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
    lay = oracle.layout(128, 128, 4, 4, 0)
    dK, dV, dR = dev.put(Kh), dev.put(Vh), dev.alloc(lay.bytes)
    for iters in (16, 0, 1, 5):
        sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dK, dV, 128, 1, 1, iters, dR, None), "sjk_hip_seal")
        got = dev.get(dR, lay.bytes, np.uint8)
        assert np.array_equal(got, oracle_seal(oracle, lay, Kh, Vh, 128, iters)), "iters=%d" % iters


def test_c1_round_trip_mse(oracle, lib, dev):
    """configs[0]'s round trip on the device: seal the group, decode it with sjk_hip_decode; the record and the
    decoded rows equal the oracle's bit for bit, so the round-trip MSE equals the oracle's (which equals the
    reference's: test_c1_round_trip_mse_matches_reference)."""
    K, V = inputs.kv_rows_c1(seed=0)
    Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
    lay = oracle.layout(128, 128, 4, 4, 0)
    dK, dV, dR = dev.put(Kh), dev.put(Vh), dev.alloc(lay.bytes)
    sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dK, dV, 128, 1, 1, 16, dR, None), "sjk_hip_seal")
    rec = dev.get(dR, lay.bytes, np.uint8)
    assert np.array_equal(rec, oracle_seal(oracle, lay, Kh, Vh, 128))
    dk, dv = dev.alloc(128 * 128 * 4), dev.alloc(128 * 128 * 4)
    sjk.check(lib.sjk_hip_decode(C.byref(play(lay)), dR, 1, dk, dv, None), "sjk_hip_decode")
    gk = dev.get(dk, 128 * 128 * 4, np.float32).reshape(128, 128)
    gv = dev.get(dv, 128 * 128 * 4, np.float32).reshape(128, 128)
    ok, ov = np.zeros((128, 128), np.float32), np.zeros((128, 128), np.float32)
    for t in range(128):
        oracle.decode_k_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(ok[t], cabi.f32p))
        oracle.decode_v_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(ov[t], cabi.f32p))
    assert np.array_equal(gk.view(np.uint32), ok.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), ov.view(np.uint32))
    assert inputs.round_trip_mse(Kh, gk) == inputs.round_trip_mse(Kh, ok)
    assert inputs.round_trip_mse(Vh, gv) == inputs.round_trip_mse(Vh, ov)


def test_seal_edge_inputs(oracle, lib, dev):
    """All-zero group, constant channels, signed zeros, and fp16 extremes (subnormals, +-65504)."""
    D, G = 256, 128
    rng = np.random.default_rng(7)
    cases = []
    cases.append((np.zeros((G, D), np.float32), np.zeros((G, D), np.float32)))
    k = rng.standard_normal((G, D)).astype(np.float32)
    k[:, 10] = 3.0
    k[5, :] = 0.0
    k[6, :] = -0.0
    cases.append((k, -k))
    k = rng.standard_normal((G, D)).astype(np.float32) * np.float32(1e-6)   # fp16 subnormals
    v = rng.standard_normal((G, D)).astype(np.float32)
    v[0, :] = 65504.0
    v[1, :] = -65504.0
    cases.append((k, v))
    for bk, bv, body in ((4, 4, 0), (3, 2, 1)):
        lay = oracle.layout(D, G, bk, bv, body)
        for K, V in cases:
            Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
            dK, dV, dR = dev.put(Kh), dev.put(Vh), dev.alloc(lay.bytes)
            sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dK, dV, D, 1, 1, 16, dR, None), "sjk_hip_seal")
            assert np.array_equal(dev.get(dR, lay.bytes, np.uint8), oracle_seal(oracle, lay, Kh, Vh, D))


NF_BODIES = [(4, 4, 0), (3, 2, 1), (3, 3, 1), (3, 3, 0), (2, 2, 1)]
MIXED_SIGN_NAN = ("scattered", "nan_first")    # tiles holding NaNs of both signs (inputs.nonfinite_groups)


@pytest.mark.parametrize("bk,bv,body", NF_BODIES, ids=["%d/%d%s" % (a, b, "t" if c else "s") for a, b, c in NF_BODIES])
def test_seal_nonfinite_inputs(oracle, lib, dev, bk, bv, body):
    """+-inf, +-quiet NaN, +-signalling NaN and NaN payloads in K and V (inputs.nonfinite_groups: scattered, lone
    infinities, all-inf rows of both signs, a NaN first in a row, all-inf and all-NaN tiles) sealed on the device in
    one launch, D = 256 and 128. Payload codes and every non-NaN scale byte for byte against the oracle; a NaN scale
    is NaN on both sides, and has the oracle's sign wherever the tile's NaNs all have one sign (the reference leaves
    that sign to the operand order its compiler chose where NaNs of both signs meet, sj_kvarn.h:943-1012)."""
    for D in (256, 128):
        lay = oracle.layout(D, 128, bk, bv, body)
        cases = inputs.nonfinite_groups(D, seed=D + bk)
        NG = len(cases)
        K = np.ascontiguousarray(np.concatenate([k for _, k, _ in cases]))
        V = np.ascontiguousarray(np.concatenate([v for _, _, v in cases]))
        dK, dV, dR = dev.put(K), dev.put(V), dev.alloc(NG * lay.bytes)
        sjk.check(lib.sjk_hip_seal(C.byref(play(lay)), dK, dV, D, 1, NG, 16, dR, None), "sjk_hip_seal")
        got = dev.get(dR, NG * lay.bytes, np.uint8).reshape(NG, lay.bytes)
        dk, dv = dev.alloc(NG * 128 * D * 4), dev.alloc(NG * 128 * D * 4)
        sjk.check(lib.sjk_hip_decode(C.byref(play(lay)), dR, NG, dk, dv, None), "sjk_hip_decode")
        rk = dev.get(dk, NG * 128 * D * 4, np.float32).reshape(NG, 128, D)
        rv = dev.get(dv, NG * 128 * D * 4, np.float32).reshape(NG, 128, D)
        row = np.zeros(D, np.float32)
        for g, (name, k, v) in enumerate(cases):
            want = oracle_seal(oracle, lay, np.ascontiguousarray(k).reshape(-1), np.ascontiguousarray(v).reshape(-1), D)
            bad = inputs.record_mismatch(lay, got[g], want)
            say("D=%d %d/%d%s %s: %d bytes differ up to NaN sign, %d exactly" % (
                D, bk, bv, "t" if body else "s", name, bad.size, int((got[g] != want).sum())))
            assert bad.size == 0, (D, name, bad[:8])
            if name not in MIXED_SIGN_NAN:
                assert np.array_equal(got[g], want), (D, name, np.nonzero(got[g] != want)[0][:8])
            rec = np.ascontiguousarray(got[g])
            for t in range(0, 128, 9):
                for fn, dec in ((oracle.decode_k_row, rk), (oracle.decode_v_row, rv)):
                    fn(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(row, cabi.f32p))
                    assert inputs.floats_equal_nan_unsigned(dec[g, t], row).all(), (D, name, t)
                    if name not in MIXED_SIGN_NAN:
                        assert np.array_equal(dec[g, t].view(np.uint32), row.view(np.uint32)), (D, name, t)


def test_stage_nonfinite_rows(oracle, lib, dev):
    """tq6_0 and fp16 staging of rows holding +-inf and NaNs (inputs.nonfinite_rows), and their unstaging: codes
    and finite norms byte for byte (a block with an infinity has an infinite norm and its infinite value takes
    level 63, sj_kvarn.h:1211-1247), NaN norms and NaN values NaN on both sides."""
    for D in (256, 128):
        n = 48
        x = inputs.nonfinite_rows(n, D, seed=D)
        dx = dev.put(x)
        rb = (D // 128) * 98
        want_q = np.zeros((n, rb), np.uint8)
        for r in range(n):
            oracle.tq6_quantize_row(cabi.ptr(x[r], cabi.f32p), want_q[r].ctypes.data, D)
        dq = dev.alloc(n * rb)
        sjk.check(lib.sjk_hip_stage(0, dx, dq, D, rb, n, None), "sjk_hip_stage")
        got_q = dev.get(dq, n * rb, np.uint8).reshape(n, rb)
        bad = inputs.tq6_mismatch(got_q, want_q)
        say("D=%d tq6: %d blocks differ up to NaN sign, %d bytes exactly" % (D, bad.size, int((got_q != want_q).sum())))
        assert bad.size == 0, bad[:8]
        # blocks whose NaNs have one sign: every byte, the NaN norm's sign included
        xb = x.reshape(n, D // 128, 128)
        one_sign = ~(np.isnan(xb) & np.signbit(xb)).any(axis=2) | ~(np.isnan(xb) & ~np.signbit(xb)).any(axis=2)
        gq, wq = got_q.reshape(n, D // 128, 98), want_q.reshape(n, D // 128, 98)
        assert np.array_equal(gq[one_sign], wq[one_sign])
        dy = dev.alloc(n * D * 4)
        sjk.check(lib.sjk_hip_unstage(0, dq, rb, dy, D, n, None), "sjk_hip_unstage")
        got_y = dev.get(dy, n * D * 4, np.float32).reshape(n, D)
        want_y = np.zeros((n, D), np.float32)
        for r in range(n):
            oracle.tq6_dequantize_row(got_q[r].ctypes.data, cabi.ptr(want_y[r], cabi.f32p), D)
        assert inputs.floats_equal_nan_unsigned(got_y, want_y).all()
        d16 = dev.alloc(n * D * 2)
        sjk.check(lib.sjk_hip_stage(1, dx, d16, D, D * 2, n, None), "sjk_hip_stage f16")
        want16 = np.zeros((n, D), np.uint16)
        for r in range(n):
            oracle.stage_row(1, cabi.ptr(x[r], cabi.f32p), want16[r].ctypes.data, D)
        got16 = dev.get(d16, n * D * 2, np.uint16).reshape(n, D)
        assert np.array_equal(got16, want16)     # a NaN keeps its own sign: sign | 0x7E00 (sj_kvarn.h:693-711)
        sjk.check(lib.sjk_hip_unstage(1, d16, D * 2, dy, D, n, None), "sjk_hip_unstage f16")
        got_y = dev.get(dy, n * D * 4, np.float32).reshape(n, D)
        for r in range(n):
            oracle.unstage_row(1, want16[r].ctypes.data, cabi.ptr(want_y[r], cabi.f32p), D)
        assert np.array_equal(got_y.view(np.uint32), want_y.view(np.uint32))


def test_rotate_and_stage_vs_oracle(oracle, lib, dev):
    """Hadamard rows, tq6_0 and fp16 staging rows, and unstaging, bit for bit (D = 128, 256, 512)."""
    rng = np.random.default_rng(3)
    for D in (128, 256, 512):
        n = 64
        x = rng.standard_normal((n, D)).astype(np.float32) * rng.lognormal(0, 2, (n, 1)).astype(np.float32)
        x[0] = 0.0
        x[1] = 1e-30
        x[2, :5] = [1e30, -1e30, 0.0, -0.0, 3.0]
        want_rot = x.copy()
        for r in range(n):
            oracle.hadamard(cabi.ptr(want_rot[r], cabi.f32p), D)
        dx = dev.put(x)
        sjk.check(lib.sjk_hip_rotate(dx, n, D, None), "sjk_hip_rotate")
        got_rot = dev.get(dx, x.nbytes, np.float32).reshape(n, D)
        assert np.array_equal(got_rot.view(np.uint32), want_rot.view(np.uint32))
        rb = (D // 128) * 98
        want_q = np.zeros((n, rb), np.uint8)
        for r in range(n):
            oracle.tq6_quantize_row(cabi.ptr(want_rot[r], cabi.f32p), want_q[r].ctypes.data, D)
        dq = dev.alloc(n * rb)
        sjk.check(lib.sjk_hip_stage(0, dx, dq, D, rb, n, None), "sjk_hip_stage")
        got_q = dev.get(dq, n * rb, np.uint8).reshape(n, rb)
        assert np.array_equal(got_q, want_q)
        dy = dev.alloc(n * D * 4)
        sjk.check(lib.sjk_hip_unstage(0, dq, rb, dy, D, n, None), "sjk_hip_unstage")
        got_y = dev.get(dy, n * D * 4, np.float32).reshape(n, D)
        want_y = np.zeros((n, D), np.float32)
        for r in range(n):
            oracle.tq6_dequantize_row(want_q[r].ctypes.data, cabi.ptr(want_y[r], cabi.f32p), D)
        assert np.array_equal(got_y.view(np.uint32), want_y.view(np.uint32))
        # fp16 staging
        d16 = dev.alloc(n * D * 2)
        sjk.check(lib.sjk_hip_stage(1, dx, d16, D, D * 2, n, None), "sjk_hip_stage f16")
        want16 = np.zeros((n, D * 2), np.uint8)
        for r in range(n):
            oracle.stage_row(1, cabi.ptr(want_rot[r], cabi.f32p), want16[r].ctypes.data, D)
        assert np.array_equal(dev.get(d16, n * D * 2, np.uint8).reshape(n, D * 2), want16)


def test_hadamard_every_power_of_two(oracle, lib, dev):
    """sj_kvarn_hadamard / rotate_heads / sjk_hip_rotate at lengths outside the row kernel's widths (the LDS
    kernel up to 8192, one launch per stage beyond), bit for bit against the oracle's butterfly (sj_kvarn.h:735-759);
    a length that is not a power of two leaves the row as it is."""
    rng = np.random.default_rng(17)
    for n in (1, 2, 4, 32, 64, 1024, 8192, 16384, 65536):
        x = (rng.standard_normal(n) * rng.lognormal(0, 3)).astype(np.float32)
        want = x.copy()
        oracle.hadamard(cabi.ptr(want, cabi.f32p), n)
        got = x.copy()
        lib.sj_kvarn_hadamard(cabi.ptr(got, cabi.f32p), n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n
    for hd, nh in ((32, 5), (64, 3), (1024, 4), (32768, 2)):
        x = rng.standard_normal((nh, hd)).astype(np.float32)
        want = x.copy()
        oracle.rotate_heads(cabi.ptr(want, cabi.f32p), nh, hd)
        got = x.copy()
        lib.sj_kvarn_rotate_heads(cabi.ptr(got, cabi.f32p), nh, hd)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), hd
        dx = dev.put(x)
        sjk.check(lib.sjk_hip_rotate(dx, nh, hd, None), "sjk_hip_rotate")
        assert np.array_equal(dev.get(dx, x.nbytes, np.float32).reshape(nh, hd).view(np.uint32), want.view(np.uint32))
    x = rng.standard_normal(96).astype(np.float32)
    y = x.copy()
    lib.sj_kvarn_hadamard(cabi.ptr(y, cabi.f32p), 96)
    assert np.array_equal(x, y)
    assert lib.sjk_hip_rotate(dev.put(x), 1, 96, None) == -100


def test_fold_rotation_into_projection_weights(oracle, lib, dev):
    """sjk_hip_fold_rotation_out / _in: every folded head block of W_q/W_k/W_v (a column's head_dim values, strided)
    and of W_o (a row's head segment) is bit for bit the oracle's sj_kvarn_hadamard of it (sj_kvarn.h:735-752), and
    the folded projections give the rotated q and accept the rotated output: W' x = rotate_heads(W x) and
    W_o' rotate_heads(o) = W_o o, within fp32 rounding of the products (float64 references)."""
    rng = np.random.default_rng(23)
    for nh, D, cols in ((4, 256, 37), (16, 128, 5), (2, 64, 1)):
        W = rng.standard_normal((nh * D, cols)).astype(np.float32)
        dW = dev.put(W)
        sjk.check(lib.sjk_hip_fold_rotation_out(dW, nh, D, cols, None), "fold_rotation_out")
        got = dev.get(dW, W.nbytes, np.float32).reshape(nh * D, cols)
        for h in range(nh):
            for c in range(cols):
                want = W[h * D:(h + 1) * D, c].copy()
                oracle.hadamard(cabi.ptr(want, cabi.f32p), D)
                assert np.array_equal(got[h * D:(h + 1) * D, c].view(np.uint32), want.view(np.uint32)), (nh, D, h, c)
        x = rng.standard_normal(cols)
        y = W.astype(np.float64) @ x                                   # W x, then the rotation per head
        H = np.array([[(-1.0) ** bin(i & j).count("1") for j in range(D)] for i in range(D)]) / np.sqrt(D)
        want = np.concatenate([H @ y[h * D:(h + 1) * D] for h in range(nh)])
        err = np.abs(got.astype(np.float64) @ x - want)
        assert np.all(err <= 1e-5 * (np.abs(W).astype(np.float64) @ np.abs(x) + 1e-30)), err.max()
        # the output side: W_o [rows][nh * D]
        rows = 7
        Wo = rng.standard_normal((rows, nh * D)).astype(np.float32)
        dWo = dev.put(Wo)
        sjk.check(lib.sjk_hip_fold_rotation_in(dWo, rows, nh, D, None), "fold_rotation_in")
        goto = dev.get(dWo, Wo.nbytes, np.float32).reshape(rows, nh * D)
        wanto = Wo.copy()
        oracle.rotate_heads(cabi.ptr(wanto, cabi.f32p), rows * nh, D)
        assert np.array_equal(goto.view(np.uint32), wanto.view(np.uint32)), (nh, D)
        o = rng.standard_normal(nh * D)
        o_rot = np.concatenate([H @ o[h * D:(h + 1) * D] for h in range(nh)])
        err = np.abs(goto.astype(np.float64) @ o_rot - Wo.astype(np.float64) @ o)
        assert np.all(err <= 1e-5 * (np.abs(Wo).astype(np.float64) @ np.abs(o) + 1e-30)), err.max()
    dW = dev.put(np.zeros(96, np.float32))
    assert lib.sjk_hip_fold_rotation_out(dW, 1, 96, 1, None) == -100
    assert lib.sjk_hip_fold_rotation_in(dW, 1, 1, 96, None) == -100


def test_record_helpers_vs_oracle(oracle, lib, dev):
    """record_scores / record_accum_v (sequential fp32, sj_kvarn.h:1288-1311) are bit-exact."""
    D, G = 256, 128
    K, V = inputs.kv_rows(G, 1, D, seed=9)
    Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
    for bk, bv, body in ((4, 4, 0), (3, 3, 1)):
        lay = oracle.layout(D, G, bk, bv, body)
        rec = oracle_seal(oracle, lay, Kh, Vh, D)
        q = np.random.default_rng(1).standard_normal(D).astype(np.float32)
        w = np.random.default_rng(2).random(G).astype(np.float32)
        acc0 = np.random.default_rng(3).standard_normal(D).astype(np.float32)
        want_s = np.zeros(G, np.float32)
        oracle.record_scores(C.byref(lay), cabi.ptr(rec), cabi.ptr(q, cabi.f32p), 100, cabi.ptr(want_s, cabi.f32p))
        want_a = acc0.copy()
        oracle.record_accum_v(C.byref(lay), cabi.ptr(rec), cabi.ptr(w, cabi.f32p), 100, cabi.ptr(want_a, cabi.f32p))
        dr, dq, dw, ds, da = dev.put(rec), dev.put(q), dev.put(w), dev.alloc(G * 4), dev.put(acc0)
        sjk.check(lib.sjk_hip_record_scores(C.byref(play(lay)), dr, dq, 100, ds, None), "record_scores")
        sjk.check(lib.sjk_hip_record_accum_v(C.byref(play(lay)), dr, dw, 100, da, None), "record_accum_v")
        assert np.array_equal(dev.get(ds, 400, np.float32).view(np.uint32), want_s[:100].view(np.uint32))
        assert np.array_equal(dev.get(da, D * 4, np.float32).view(np.uint32), want_a.view(np.uint32))


def test_dropin_host_api(oracle, lib):
    """The sj_kvarn.h-named calls on host arrays (a drop-in for the reference header) match the oracle."""
    D, G = 256, 128
    lay = oracle.layout(D, G, 3, 2, 1)
    K = np.zeros(D * G, np.uint16)
    V = np.zeros(D * G, np.uint16)
    oracle.vec_fill_group(D, G, 4, cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p))
    want = oracle_seal(oracle, lay, K, V, D)
    got = np.zeros(lay.bytes, np.uint8)
    pl = play(lay)
    lib.sj_kvarn_seal_group(C.byref(pl), cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p), D, 16, cabi.ptr(got), None)
    assert np.array_equal(got, want)
    a, b = np.zeros(D, np.float32), np.zeros(D, np.float32)
    for t in (0, 77, 127):
        lib.sj_kvarn_decode_v_row(C.byref(pl), cabi.ptr(got), t, cabi.ptr(a, cabi.f32p))
        oracle.decode_v_row(C.byref(lay), cabi.ptr(want), t, cabi.ptr(b, cabi.f32p))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    x = np.random.default_rng(5).standard_normal(D).astype(np.float32)
    xa, xb = x.copy(), x.copy()
    lib.sj_kvarn_hadamard(cabi.ptr(xa, cabi.f32p), D)
    oracle.hadamard(cabi.ptr(xb, cabi.f32p), D)
    assert np.array_equal(xa.view(np.uint32), xb.view(np.uint32))
    qa, qb = np.zeros(196, np.uint8), np.zeros(196, np.uint8)
    lib.sj_kvarn_stage_row(0, cabi.ptr(xa, cabi.f32p), qa.ctypes.data, D)
    oracle.stage_row(0, cabi.ptr(xb, cabi.f32p), qb.ctypes.data, D)
    assert np.array_equal(qa, qb)
