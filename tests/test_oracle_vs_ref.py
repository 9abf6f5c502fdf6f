"""The oracle against the reference compiled from its own header (oracle/_ref), on fresh seeded inputs.

The golden vectors pin one input per config; this widens the check to more seeds, to the BASELINE shape
(D = 256, several heads), to the per-layer cache (store / seal / attend) and to the sequence state stream.
Skipped where oracle/_ref is not built.
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import cabi

BODIES = [(4, 4, 0), (3, 3, 1), (3, 2, 1), (2, 2, 1), (4, 3, 0), (3, 3, 0), (4, 2, 0), (2, 4, 0), (3, 2, 0), (2, 2, 0)]


def seal(api, lay, K, V, stride=None):
    D = lay.D
    rec = np.zeros(lay.bytes, np.uint8)
    work = np.zeros(api.seal_workspace_bytes(C.byref(lay)), np.uint8)
    api.seal_group(C.byref(lay), cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p), stride or D, 16, cabi.ptr(rec),
                   work.ctypes.data_as(C.c_void_p))
    return rec


@pytest.mark.parametrize("bk,bv,body", BODIES)
def test_seal_records_match_reference(oracle, ref, bk, bv, body):
    D = 256
    lay = oracle.layout(D, 128, bk, bv, body)
    assert oracle.seal_workspace_bytes(C.byref(lay)) == ref.seal_workspace_bytes(C.byref(lay))
    for seed in (7, 1234):
        K = np.zeros(D * 128, np.uint16)
        V = np.zeros(D * 128, np.uint16)
        oracle.vec_fill_group(D, 128, seed, cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p))
        a, b = seal(oracle, lay, K, V), seal(ref, lay, K, V)
        assert np.array_equal(a, b), "seed %d" % seed
        ra, rb = np.zeros(D, np.float32), np.zeros(D, np.float32)
        for t in (0, 17, 127):
            for fa, fb in ((oracle.decode_k_row, ref.decode_k_row), (oracle.decode_v_row, ref.decode_v_row)):
                fa(C.byref(lay), cabi.ptr(a), t, cabi.ptr(ra, cabi.f32p))
                fb(C.byref(lay), cabi.ptr(a), t, cabi.ptr(rb, cabi.f32p))
                assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32))


def minmax4_mse(x_bits, axis):
    """MSE of a plain 4-bit min-max quantizer (round to nearest on 16 levels between the extremes along axis) on
    fp16 rows [128][128]: the yardstick for the codec's round trip"""
    x = np.asarray(x_bits, np.uint16).view(np.float16).astype(np.float64).reshape(128, 128)
    lo, hi = x.min(axis=axis, keepdims=True), x.max(axis=axis, keepdims=True)
    st = np.where(hi > lo, (hi - lo) / 15.0, 1.0)
    d = np.clip(np.round((x - lo) / st), 0, 15) * st + lo
    return float(np.mean((d - x) ** 2))


def test_c1_round_trip_mse_matches_reference(oracle, ref):
    """seal one 128-token group (1 KV head, D = 128, 4/4, K channels 3 and 77 x12) and decode it. The
    record and every decoded row equal the reference's, so its round-trip MSE does (the reference publishes no
    figure for it). Independent yardstick: a plain 4-bit min-max quantizer along the codec's own axes (K per
    channel, V per token) on the same rows; the codec's scales and variance balance must do at least as well, and
    no 4-bit code does better than about half of it (K: 0.0261 against 0.0275, V: 0.00967 against 0.0101)."""
    import inputs
    K, V = inputs.kv_rows_c1(seed=0)
    Kh, Vh = inputs.f16_bits(K).reshape(-1), inputs.f16_bits(V).reshape(-1)
    lay = oracle.layout(128, 128, 4, 4, 0)
    a, b = seal(oracle, lay, Kh, Vh), seal(ref, lay, Kh, Vh)
    assert np.array_equal(a, b)
    dec = {}
    for name, api in (("oracle", oracle), ("ref", ref)):
        dk, dv = np.zeros((128, 128), np.float32), np.zeros((128, 128), np.float32)
        for t in range(128):
            api.decode_k_row(C.byref(lay), cabi.ptr(a), t, cabi.ptr(dk[t], cabi.f32p))
            api.decode_v_row(C.byref(lay), cabi.ptr(a), t, cabi.ptr(dv[t], cabi.f32p))
        dec[name] = (dk, dv)
    for i in range(2):
        assert np.array_equal(dec["oracle"][i].view(np.uint32), dec["ref"][i].view(np.uint32))
    dk, dv = dec["oracle"]
    for x, d, axis in ((Kh, dk, 0), (Vh, dv, 1)):
        mse, rel = inputs.round_trip_mse(x, d)
        naive = minmax4_mse(x, axis)
        assert 0.5 * naive < mse <= naive, (mse, naive)
        assert rel < 0.02, rel


def test_seal_signed_zero_and_constant_rows(oracle, ref):
    """Edge cases the ternary min/max and the zero branches decide: all-zero tiles, +-0 mixes, constant rows."""
    D = 256
    rng = np.random.default_rng(3)
    for bk, bv, body in [(4, 4, 0), (3, 2, 1), (3, 3, 1)]:
        lay = oracle.layout(D, 128, bk, bv, body)
        K = np.zeros(D * 128, np.uint16)
        V = np.where(rng.random(D * 128) < 0.5, 0x8000, 0).astype(np.uint16)      # +0 / -0
        assert np.array_equal(seal(oracle, lay, K, V), seal(ref, lay, K, V))
        K = np.full(D * 128, 0x3C00, np.uint16)                                    # constant 1.0
        V = rng.integers(0, 0x7800, D * 128).astype(np.uint16) | (rng.integers(0, 2, D * 128).astype(np.uint16) << 15)
        assert np.array_equal(seal(oracle, lay, K, V), seal(ref, lay, K, V))


def test_tq6_rows_match_reference(oracle, ref):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(64 * 256) * rng.lognormal(0, 1, 64).repeat(256)).astype(np.float32)
    x[:256] = 0
    x[256:384] = -0.0
    x[512] = np.float32(1e-30)
    for staging, nb in ((0, 196), (1, 512)):
        a = np.zeros(64 * nb, np.uint8)
        b = np.zeros(64 * nb, np.uint8)
        for r in range(64):
            oracle.stage_row(staging, cabi.ptr(x[r * 256:], cabi.f32p), a[r * nb:].ctypes.data, 256)
            ref.stage_row(staging, cabi.ptr(x[r * 256:], cabi.f32p), b[r * nb:].ctypes.data, 256)
        assert np.array_equal(a, b)


NONFINITE_BODIES = [(4, 4, 0), (3, 2, 1), (3, 3, 1), (3, 3, 0), (2, 2, 1)]


@pytest.mark.parametrize("bk,bv,body", NONFINITE_BODIES)
def test_seal_nonfinite_inputs_match_reference(oracle, ref, bk, bv, body):
    """+-inf, +-quiet NaN, +-signalling NaN and NaN payloads in K and V (inputs.nonfinite_groups): record bytes
    and decoded rows. Tiles whose NaNs all have one sign (the infinity cases, where the seal itself makes NaNs
    from inf - inf, and the all-NaN tiles) give the same bytes in both builds. Where NaNs of both signs meet in
    one add or multiply, the sign of the result is the operand order gcc chose, which differs between the two
    builds (IEEE 754 leaves it unspecified): there the records agree up to the sign of NaN scales, and nowhere
    else (payload codes exactly, every non-NaN scale exactly)."""
    import inputs
    for D in (256, 128):
        lay = oracle.layout(D, 128, bk, bv, body)
        for name, K, V in inputs.nonfinite_groups(D, seed=D + bk):
            K, V = np.ascontiguousarray(K).reshape(-1), np.ascontiguousarray(V).reshape(-1)
            a, b = seal(oracle, lay, K, V), seal(ref, lay, K, V)
            bad = inputs.record_mismatch(lay, a, b)
            assert bad.size == 0, (D, name, bad[:8])
            if name not in ("scattered", "nan_first"):
                assert np.array_equal(a, b), (D, name, np.nonzero(a != b)[0][:8])
            ra, rb = np.zeros(D, np.float32), np.zeros(D, np.float32)
            for t in (0, 5, 127):
                for fa, fb in ((oracle.decode_k_row, ref.decode_k_row), (oracle.decode_v_row, ref.decode_v_row)):
                    fa(C.byref(lay), cabi.ptr(a), t, cabi.ptr(ra, cabi.f32p))
                    fb(C.byref(lay), cabi.ptr(a), t, cabi.ptr(rb, cabi.f32p))
                    assert inputs.floats_equal_nan_unsigned(ra, rb).all(), (D, name, t)
                    if name not in ("scattered", "nan_first"):
                        assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32)), (D, name, t)


def test_tq6_nonfinite_rows_match_reference(oracle, ref):
    """tq6_0 and fp16 staging of rows holding +-inf and NaNs (a block with an infinity has an infinite norm and
    its infinite value quantizes as NaN, level 63; a block with a NaN has a NaN norm), and unstaging them."""
    import inputs
    x = inputs.nonfinite_rows(48, 256, seed=4)
    for staging, nb in ((0, 196), (1, 512)):
        a = np.zeros(48 * nb, np.uint8)
        b = np.zeros(48 * nb, np.uint8)
        for r in range(48):
            oracle.stage_row(staging, cabi.ptr(x[r], cabi.f32p), a[r * nb:].ctypes.data, 256)
            ref.stage_row(staging, cabi.ptr(x[r], cabi.f32p), b[r * nb:].ctypes.data, 256)
        assert np.array_equal(a, b), staging
        ya, yb = np.zeros(256, np.float32), np.zeros(256, np.float32)
        for r in range(48):
            oracle.unstage_row(staging, a[r * nb:].ctypes.data, cabi.ptr(ya, cabi.f32p), 256)
            ref.unstage_row(staging, a[r * nb:].ctypes.data, cabi.ptr(yb, cabi.f32p), 256)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (staging, r)
    # the level of a NaN value is 63 (the binary search never moves left): a block holding one +inf
    blk = np.zeros(98, np.uint8)
    row = np.ones(128, np.float32)
    row[7] = np.inf
    oracle.tq6_quantize_row(cabi.ptr(row, cabi.f32p), blk.ctypes.data, 128)
    code7 = ((blk[2 + 3] >> 4) & 15) | (((blk[66 + 1] >> 6) & 3) << 4)
    assert code7 == 63 and blk[:2].view(np.uint16)[0] == 0x7C00


def test_hadamard_matches_reference(oracle, ref):
    rng = np.random.default_rng(5)
    for n in (32, 128, 256, 1024):
        x = rng.standard_normal(n).astype(np.float32)
        a, b = x.copy(), x.copy()
        oracle.hadamard(cabi.ptr(a, cabi.f32p), n)
        ref.hadamard(cabi.ptr(b, cabi.f32p), n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _grow_layer(api, cfg, N, seed):
    L = cabi.Layer()
    assert api.layer_init(C.byref(L), C.byref(cfg)) == 0
    p = cabi.Policy()
    api.policy_init(C.byref(p), cfg.sink, cfg.tail, cfg.tail_max, cfg.group, cfg.flush_chunk)
    rng = np.random.default_rng(seed)
    H, D = cfg.n_head_kv, cfg.head_dim
    x = rng.standard_normal((N, 2, H * D)).astype(np.float32)
    for pos in range(0, N, 16):
        if api.policy_begin_ubatch(C.byref(p), pos, 16) > p.B:
            api.layer_seal(C.byref(L), p.B, p.B_pending)
        api.policy_commit(C.byref(p))
        for i in range(pos, min(N, pos + 16)):
            api.layer_store(C.byref(L), i, cabi.ptr(x[i, 0], cabi.f32p), cabi.ptr(x[i, 1], cabi.f32p))
    return L, p


@pytest.mark.parametrize("bk,bv", [(4, 4), (3, 2)])
def test_layer_attention_matches_reference(oracle, ref, bk, bv):
    cfg = oracle.config_default(256, 2, 2048, 64)
    cfg.bits_k, cfg.bits_v, cfg.tail, cfg.tail_max = bk, bv, 256, 512
    N = 1100
    La, pa = _grow_layer(oracle, cfg, N, 9)
    Lb, pb = _grow_layer(ref, cfg, N, 9)
    assert pa.B == pb.B and pa.B > 128
    nbody = La.n_groups * 2 * La.lay.bytes
    assert np.array_equal(np.ctypeslib.as_array(La.body, (nbody,)), np.ctypeslib.as_array(Lb.body, (nbody,)))
    rng = np.random.default_rng(1)
    q = rng.standard_normal(256).astype(np.float32)
    oa, ob = np.zeros(256, np.float32), np.zeros(256, np.float32)
    for h, qpos in ((0, N - 1), (1, N - 1), (1, 500), (0, 60)):
        oracle.layer_attend_row(C.byref(La), pa.B, N, cabi.ptr(q, cabi.f32p), h, qpos, 0.0625, cabi.ptr(oa, cabi.f32p))
        ref.layer_attend_row(C.byref(Lb), pb.B, N, cabi.ptr(q, cabi.f32p), h, qpos, 0.0625, cabi.ptr(ob, cabi.f32p))
        assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
    oracle.layer_free(C.byref(La))
    ref.layer_free(C.byref(Lb))


@pytest.mark.parametrize("D,bk,bv,body", [(256, 4, 4, 0), (128, 4, 4, 0), (256, 3, 2, 1), (256, 2, 2, 1), (256, 4, 2, 0)])
def test_record_scores_and_accum_v_match_reference(oracle, ref, D, bk, bv, body):
    """sjo_record_scores / sjo_record_accum_v against the reference's sj_kvarn_record_scores /
    sj_kvarn_record_accum_v (sj_kvarn.h:1288-1311) bit for bit: several token counts n (including 0, 1 and G),
    queries and weights of mixed scale, and a non-zero starting accumulator that must be added to, not
    overwritten. A float64 dot over the decoded rows bounds both (a dropped term or a wrong row fails it)."""
    lay = oracle.layout(D, 128, bk, bv, body)
    K = np.zeros(D * 128, np.uint16)
    V = np.zeros(D * 128, np.uint16)
    oracle.vec_fill_group(D, 128, 77 + D + bk, cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p))
    rec = seal(ref, lay, K, V)
    rng = np.random.default_rng(D + 10 * bk + bv)
    rows_k = np.zeros((128, D), np.float32)
    rows_v = np.zeros((128, D), np.float32)
    for t in range(128):
        ref.decode_k_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(rows_k[t], cabi.f32p))
        ref.decode_v_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(rows_v[t], cabi.f32p))
    for n in (0, 1, 7, 64, 127, 128):
        q = (rng.standard_normal(D) * rng.lognormal(0, 2, D)).astype(np.float32)
        sa = np.full(128, 7.0, np.float32)
        sb = np.full(128, 7.0, np.float32)
        oracle.record_scores(C.byref(lay), cabi.ptr(rec), cabi.ptr(q, cabi.f32p), n, cabi.ptr(sa, cabi.f32p))
        ref.record_scores(C.byref(lay), cabi.ptr(rec), cabi.ptr(q, cabi.f32p), n, cabi.ptr(sb, cabi.f32p))
        assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32)), n
        assert np.all(sa[n:] == 7.0), "scores past n must be left alone"
        exact = rows_k[:n].astype(np.float64) @ q.astype(np.float64)
        mag = np.abs(rows_k[:n].astype(np.float64)) @ np.abs(q.astype(np.float64))
        assert np.all(np.abs(sa[:n] - exact) <= 1e-5 * mag + 1e-30)
        w = rng.random(128).astype(np.float32) * np.float32(3.0)
        acc0 = rng.standard_normal(D).astype(np.float32) * np.float32(5.0)
        aa, ab = acc0.copy(), acc0.copy()
        oracle.record_accum_v(C.byref(lay), cabi.ptr(rec), cabi.ptr(w, cabi.f32p), n, cabi.ptr(aa, cabi.f32p))
        ref.record_accum_v(C.byref(lay), cabi.ptr(rec), cabi.ptr(w, cabi.f32p), n, cabi.ptr(ab, cabi.f32p))
        assert np.array_equal(aa.view(np.uint32), ab.view(np.uint32)), n
        exact = acc0.astype(np.float64) + w[:n].astype(np.float64) @ rows_v[:n].astype(np.float64)
        mag = np.abs(acc0.astype(np.float64)) + w[:n].astype(np.float64) @ np.abs(rows_v[:n].astype(np.float64))
        assert np.all(np.abs(aa - exact) <= 1e-5 * mag + 1e-30)


def test_reference_kl_check_output_is_the_fixture():
    """tests/golden/expected_kl.txt is the output of the reference's own KL sanity check (tests/test_kl.c, compiled
    from its sources by oracle/Makefile); the device test compares its figures with it."""
    exe = os.path.join(cabi.ROOT, "oracle", "_ref", "test_kl")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_kl (the reference's KL check) is not built here")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.strip().endswith("PASS")
    assert out.stdout == open(os.path.join(cabi.ROOT, "tests", "golden", "expected_kl.txt")).read()


@pytest.mark.parametrize("name", ["test_vectors", "test_policy", "test_fp16"])
def test_reference_own_tests_pass(name):
    """The reference's own C tests (built from its sources into oracle/_ref by oracle/Makefile) pass on this
    machine: the golden vectors the oracle is pinned to are the reference's, checked by the reference itself
    (test_vectors reads the reference's tests/expected_vectors.txt, so it runs in the reference tree). test_state
    (~2 minutes) is left out; its 5 stream hashes pin the oracle in test_oracle_state.py."""
    exe = os.path.join(cabi.ROOT, "oracle", "_ref", name)
    ref_dir = "/root/reference"
    if not os.path.exists(exe) or not os.path.isdir(ref_dir):
        pytest.skip("the reference's tests are not built here (oracle/_ref) or its tree is absent")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300, cwd=ref_dir)
    assert out.returncode == 0, out.stdout[-2000:]
    assert "PASS" in out.stdout.strip().splitlines()[-1]
