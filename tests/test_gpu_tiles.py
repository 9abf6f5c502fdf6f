"""Attention at every query shape the reference takes (sj_kvarn_cuda.cuh:102-135: any n_q x n_head): the query
rows of a KV head (n_q positions x the GQA group) are cut into 16-row tiles, up to 8 per launch, on the matrix-core
kernels (every scalar and trellis body at D = 128 and 256).

Bar: |gpu - oracle| <= 1e-3 + 1e-3 |oracle| per value against the oracle's position-ordered loop
(sj_kvarn.h:1535-1564), the BASELINE tolerance; the reference's own device test (tests/test_cuda.cu:84-135)
also reports the relative L2 error of each row, which is bounded here by 1e-3.
"""
import ctypes as C
import os
import sys
import threading

import numpy as np
import pytest

import cabi
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

from test_gpu_layer import device_context, make_pair  # noqa: E402

pytestmark = pytest.mark.gpu
ATOL = RTOL = 1e-3
N_THREADS = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.fixture(scope="module")
def dev():
    d = sjk.Device()
    yield d
    d.free_all()


def oracle_rows(oracle, OL, B, N, q, qpos0, scale, rows):
    """the oracle's layer_attend_row for (iq, hq) pairs, on host threads"""
    n_q, n_head, D = q.shape
    gq = n_head // OL.cfg.n_head_kv
    out = {}

    def work(k):
        for iq, hq in rows[k::N_THREADS]:
            o = np.zeros(D, np.float32)
            qq = np.ascontiguousarray(q[iq, hq])
            oracle.layer_attend_row(C.byref(OL), B, N, cabi.ptr(qq, cabi.f32p), hq // gq, qpos0 + iq, scale,
                                    cabi.ptr(o, cabi.f32p))
            out[(iq, hq)] = o

    ths = [threading.Thread(target=work, args=(k,)) for k in range(N_THREADS)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    return out


def check_rows(got, want):
    worst, worst_l2 = 0.0, 0.0
    for (iq, hq), w in want.items():
        g = got[iq, hq]
        err = np.abs(g - w)
        assert np.all(err <= ATOL + RTOL * np.abs(w)), "row (%d,%d) max abs err %g" % (iq, hq, err.max())
        worst = max(worst, float((err / (ATOL + RTOL * np.abs(w))).max()))
        n2 = float(np.sum(w.astype(np.float64) ** 2))
        worst_l2 = max(worst_l2, float(np.sqrt(np.sum((g - w).astype(np.float64) ** 2) / (n2 if n2 > 0 else 1.0))))
    return worst, worst_l2


def attend(lib, dev, view, B, N, qpos0, q, scale):
    dq, do = dev.put(q), dev.alloc(q.nbytes)
    sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, qpos0, q.shape[0], q.shape[1], dq, scale, do, None), "attend")
    got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
    dev.free(dq)
    dev.free(do)
    return got


def test_reference_device_test_shape(oracle, lib):
    """The reference's own device attention test (tests/test_cuda.cu:84-135): D = 256, 2 KV heads, 3/3 trellis
    body, tail 256 / tail_max 512, 1200 positions stored in ubatches of 16 through the host API, then the last
    16 positions with 4 query heads each (32 query rows per KV head: two tiles). The cache is built through
    libsjk's sj_kvarn_* calls exactly as the reference test builds its own, and must equal the oracle's
    byte for byte."""
    D, H, NPOS, NQ, HQ = 256, 2, 1200, 16, 4
    rng = np.random.default_rng(99)
    x = (rng.standard_normal((NPOS, H * D)) / 1024.0).astype(np.float32)
    q = (rng.standard_normal((NPOS, HQ, D)) / 1024.0).astype(np.float32)
    layers = []
    for api in (oracle, lib):
        cfg = (cabi.Config if api is oracle else sjk.Config).from_buffer_copy(bytes(oracle.config_default(D, H, 2048, 64)))
        cfg.bits_k, cfg.bits_v, cfg.tail, cfg.tail_max = 3, 3, 256, 512
        L = cabi.Layer() if api is oracle else sjk.Layer()
        if api is oracle:
            assert oracle.layer_init(C.byref(L), C.byref(cfg)) == 0
            pol = cabi.Policy()
            oracle.policy_init(C.byref(pol), cfg.sink, cfg.tail, cfg.tail_max, 128, 0)
            begin, commit, seal, store = (oracle.policy_begin_ubatch, oracle.policy_commit, oracle.layer_seal,
                                          oracle.layer_store)
        else:
            sjk.check(lib.sj_kvarn_layer_init(C.byref(L), C.byref(cfg)), "layer_init")
            pol = sjk.Policy()
            lib.sj_kvarn_policy_init(C.byref(pol), cfg.sink, cfg.tail, cfg.tail_max, 128, 0)
            begin, commit, seal, store = (lib.sj_kvarn_policy_begin_ubatch, lib.sj_kvarn_policy_commit,
                                          lib.sj_kvarn_layer_seal, lib.sj_kvarn_layer_store)
        for p in range(0, NPOS, 16):
            if begin(C.byref(pol), p, 16) > pol.B:
                seal(C.byref(L), pol.B, pol.B_pending)
            commit(C.byref(pol))
            for i in range(p, p + 16):
                store(C.byref(L), i, x[i].ctypes.data_as(cabi.f32p), x[(i * 7) % NPOS].ctypes.data_as(cabi.f32p))
        layers.append((L, pol))
    (OL, opol), (PL, ppol) = layers
    d = sjk.Device()
    try:
        assert opol.B == ppol.B and opol.B > 128
        for name, nb in (("sink", 128 * H * D * 4), ("ring", OL.cap * H * 2 * OL.stage_bytes),
                         ("body", (opol.B - 128) // 128 * H * OL.lay.bytes)):
            got = d.get(C.c_void_p(getattr(PL, name)), nb, np.uint8)
            want = np.ctypeslib.as_array(C.cast(getattr(OL, name), cabi.u8p), shape=(nb,))
            assert np.array_equal(got, want), name
        qpos0 = NPOS - NQ
        qq = np.ascontiguousarray(q[qpos0:])
        view = lib.sjk_layer_view(C.byref(PL))
        got = attend(lib, d, view, ppol.B, NPOS, qpos0, qq, 1.0 / 16.0)
        want = oracle_rows(oracle, OL, opol.B, NPOS, qq, qpos0, 1.0 / 16.0,
                           [(iq, hq) for iq in range(NQ) for hq in range(HQ)])
        worst, l2 = check_rows(got, want)
        say("[tiles] reference shape: worst %.4f of the tolerance, max rel L2 %.2e" % (worst, l2))
        assert l2 <= 1e-3
    finally:
        d.free_all()
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("bk,bv,body,n_q,D", [(4, 4, 0, 512, 256), (3, 3, 1, 96, 256), (4, 4, 0, 512, 128)],
                         ids=["4/4s-ubatch512", "3/3t-ubatch96", "d128-4/4s-ubatch512"])
def test_prefill_ubatch(oracle, lib, dev, bk, bv, body, n_q, D):
    """A prefill ubatch of n_q positions x 16 query heads (GQA 4:1: 4 n_q rows per KV head, many launches of 8
    tiles) at the end of a context with a sealed body and a tq6_0 tail; the positions of the ubatch are both in
    the tail and (causally masked) in the body. Sampled rows from every part of the ubatch."""
    H, S, G = 4, 128, 128
    B = S + 12 * G
    n_pos = B + 700
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 1024, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=4000 + bk)
        n_head = 16
        q = np.random.default_rng(21).standard_normal((n_q, n_head, D)).astype(np.float32)
        qpos0 = n_pos - n_q
        got = attend(lib, dev, view, B, n_pos, qpos0, q, 0.0625)
        assert np.all(np.isfinite(got))
        rng = np.random.default_rng(n_q)
        rows = sorted({(0, 0), (0, 15), (n_q - 1, 0), (n_q - 1, 15), (n_q // 2, 5)} |
                      {(int(a), int(b)) for a, b in zip(rng.integers(0, n_q, 40), rng.integers(0, n_head, 40))})
        worst, l2 = check_rows(got, oracle_rows(oracle, OL, B, n_pos, q, qpos0, 0.0625, rows))
        say("[tiles] ubatch %d: %d rows, worst %.4f of the tolerance, rel L2 %.2e" % (n_q, len(rows), worst, l2))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


SHAPES = [
    # D, H, bk, bv, body, n_q, n_head
    (128, 1, 4, 4, 0, 4, 4),        # configs[0]'s shape (1 KV head, D = 128, 4/4), decode width 4: the 4/4
    (128, 1, 4, 4, 0, 40, 4),       # the same, 160 query rows: 10 tiles, two launches     matrix-core kernel
    (128, 8, 4, 4, 0, 4, 32),       # 8 KV heads, GQA 4:1, width 4 (the common D = 128 decode shape)
    (128, 2, 3, 3, 1, 4, 8),        # trellis at D = 128
    (128, 2, 4, 2, 0, 9, 8),        # 4/2 scalar at D = 128, 36 rows per KV head: the other scalar bodies' kernel
    (256, 4, 3, 3, 0, 4, 16),       # a scalar body other than 4/4 at D = 256
    (256, 4, 4, 2, 0, 9, 16),       # 4/2 scalar, 36 rows per KV head
]


@pytest.mark.parametrize("D,H,bk,bv,body,n_q,n_head", SHAPES,
                         ids=["c1-d128-w4", "c1-d128-160rows", "d128-h8-w4", "d128-3/3t", "d128-4/2s",
                              "d256-3/3s", "d256-4/2s-36rows"])
def test_shapes_vs_oracle(oracle, lib, dev, D, H, bk, bv, body, n_q, n_head):
    S, G = 128, 128
    B = S + 5 * G
    n_pos = B + 333
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=5000 + D + bk)
        q = np.random.default_rng(31).standard_normal((n_q, n_head, D)).astype(np.float32)
        for qpos0 in (n_pos - n_q, B - n_q // 2 - 3):          # rows in the tail; rows across the body's end
            got = attend(lib, dev, view, B, n_pos, qpos0, q, 1.0 / float(np.sqrt(D)))
            rows = [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
            if len(rows) > 64:
                rows = rows[::len(rows) // 48]
            worst, _ = check_rows(got, oracle_rows(oracle, OL, B, n_pos, q, qpos0, 1.0 / float(np.sqrt(D)), rows))
            say("[tiles] D=%d H=%d %d/%d%s qpos0=%d: worst %.4f" % (D, H, bk, bv, "t" if body else "s", qpos0, worst))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 2, 1), (4, 2, 0)], ids=["4/4s", "3/2t", "4/2s"])
def test_wide_gqa_group(oracle, lib, dev, bk, bv, body):
    """32 query heads per KV head: one position's rows span two tiles (a tile boundary inside a position)."""
    D, H, S, G = 256, 2, 128, 128
    B = S + 4 * G
    n_pos = B + 300                                   # the context builder keeps the last 256 positions unsealed
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=6000 + bk)
        n_q, n_head = 3, 64
        q = np.random.default_rng(41).standard_normal((n_q, n_head, D)).astype(np.float32)
        got = attend(lib, dev, view, B, n_pos, n_pos - n_q, q, 0.0625)
        rows = [(iq, hq) for iq in range(n_q) for hq in range(0, n_head, 5)] + [(1, 31), (1, 32), (2, 63)]
        worst, _ = check_rows(got, oracle_rows(oracle, OL, B, n_pos, q, n_pos - n_q, 0.0625, rows))
        say("[tiles] gq=32 %d/%d: worst %.4f" % (bk, bv, worst))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("bk,bv,body,D", [(4, 4, 0, 256), (3, 3, 1, 256), (4, 4, 0, 128)], ids=["4/4s", "3/3t", "d128-4/4s"])
def test_small_and_edge_contexts(oracle, lib, dev, bk, bv, body, D):
    """One KV head (GQA 16:1, so 16 rows per position and several tiles at width 4) over contexts at the region
    edges on the matrix-core kernels: a single sink position, a partial sink, the sink exactly full, one tail
    position, a body that ends exactly at N (no tail), queries at the very start (causal prefixes of the sink),
    and part of the stored groups read from the ring instead of the body."""
    H, S, G = 1, 128, 128
    n_pos = S + 2 * G + 37
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        K, V = inputs.kv_rows(n_pos, H, D, seed=8800 + bk)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, 1, None), "layer_store")
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, S + 2 * G, 16, None), "commit")
        dev.sync()
        assert n_pos - S <= PL.cap
        for name, nb in (("sink", S * H * D * 4), ("ring", OL.cap * H * 2 * OL.stage_bytes),
                         ("body", 2 * H * OL.lay.bytes)):
            b = dev.get(C.c_void_p(getattr(view, name)), nb, np.uint8)
            C.memmove(getattr(OL, name), b.ctypes.data, nb)
        n_head = 16
        cases = [  # B, N, qpos0, n_q
            (0, 1, 0, 1), (0, 64, 63, 1), (S, S, S - 4, 4), (S, S + 1, S, 1), (S + 2 * G, S + 2 * G, S + 2 * G - 4, 4),
            (S + 2 * G, n_pos, 0, 4), (S + G, n_pos, n_pos - 4, 4), (S + 2 * G, n_pos, n_pos - 4, 4)]
        for B, N, qpos0, n_q in cases:
            q = np.random.default_rng(B + N + qpos0).standard_normal((n_q, n_head, D)).astype(np.float32)
            got = attend(lib, dev, view, B, N, qpos0, q, 0.0625)
            rows = [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
            worst, _ = check_rows(got, oracle_rows(oracle, OL, B, N, q, qpos0, 0.0625, rows))
            say("[tiles] H=1 D=%d %d/%d%s B=%d N=%d qpos0=%d n_q=%d: worst %.4f" % (D, bk, bv, "t" if body else "s", B,
                                                                                   N, qpos0, n_q, worst))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


WIDE = [
    # D, H, bk, bv, body, n_q, n_head, sealed groups
    (256, 4, 4, 4, 0, 5, 16, 14),   # width 5 at GQA 4:1: 20 rows per KV head, the configs[3] layout
    (128, 4, 4, 4, 0, 4, 32, 14),   # width 4 at GQA 8:1: 32 rows (the common D = 128 shape)
    (128, 4, 4, 4, 0, 4, 32, 0),    # the same with no sealed records: row slots only
    (128, 96, 4, 4, 0, 4, 768, 3),  # 96 KV heads: two CU slots per KV head for two jobs, each share raised to two
    (256, 4, 4, 4, 0, 8, 16, 14),   # 32 rows at D = 256
    (256, 4, 3, 3, 0, 5, 16, 14),   # a scalar body other than 4/4, 20 rows
    (128, 2, 4, 2, 0, 8, 8, 14),    # 4/2 at D = 128, 32 rows
    (256, 4, 3, 3, 1, 5, 16, 14),   # the 3/3 trellis body, 20 rows
]


@pytest.mark.parametrize("D,H,bk,bv,body,n_q,n_head,n_groups", WIDE,
                         ids=["4/4-d256-20rows", "4/4-d128-32rows", "4/4-d128-32rows-tail-only", "4/4-d128-32rows-96heads",
                              "4/4-d256-32rows", "3/3s-d256-20rows", "4/2s-d128-32rows", "3/3t-d256-20rows"])
def test_wide_rows_vs_oracle(oracle, lib, dev, D, H, bk, bv, body, n_q, n_head, n_groups):
    """More than 16 query rows per KV head: the 16-row tiles run side by side as the jobs of one launch, sharing its
    workgroups in proportion to their work (the 4/4 kernel, the other scalar bodies' kernel, the trellis kernel).
    Every row of the call against the oracle, for rows in the tail and rows across the body's (sink's) end; the
    second tile's rows see one position more than the first's at width 5 (the causal end of each row is its own)."""
    S, G = 128, 128
    B = S + n_groups * G
    n_pos = B + 301
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=7100 + D + bk + n_q)
        q = np.random.default_rng(33 + n_q).standard_normal((n_q, n_head, D)).astype(np.float32)
        for qpos0 in (n_pos - n_q, B - 2):                  # rows in the tail; rows across the body's (sink's) end
            got = attend(lib, dev, view, B, n_pos, qpos0, q, 1.0 / float(np.sqrt(D)))
            rows = [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
            worst, l2 = check_rows(got, oracle_rows(oracle, OL, B, n_pos, q, qpos0, 1.0 / float(np.sqrt(D)), rows))
            say("[tiles] wide D=%d H=%d %d/%d %d rows qpos0=%d: worst %.4f, rel L2 %.2e" % (
                D, H, bk, bv, n_q * n_head // H, qpos0, worst, l2))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))
