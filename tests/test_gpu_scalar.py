"""Decode attention over the scalar bodies other than 4/4 (the reference's 4/3, 3/3, 4/2, 2/4, 3/2, 2/2 vectors and
3/4, 2/3; sj_kvarn.h:771-833) at D = 128 and 256, on their matrix-core kernel (attendsc_kernel): 4-bit sides in the
fragment order, 2- and 3-bit sides token-major.

Bar: |gpu - oracle| <= 1e-3 + 1e-3 |oracle| per value against the oracle's position-ordered loop
(sj_kvarn.h:1535-1564). The records are sealed on the device and compared byte for byte with the oracle's seal
first, so the attention is checked on the reference's own bytes.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import cabi
import contexts
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

from test_gpu_layer import host_bytes, make_pair, oracle_store  # noqa: E402
from test_gpu_tiles import check_rows, oracle_rows  # noqa: E402

pytestmark = pytest.mark.gpu
ATOL = RTOL = 1e-3
BODIES = [(4, 3), (3, 3), (4, 2), (2, 4), (3, 2), (2, 2), (3, 4), (2, 3)]


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


@pytest.mark.parametrize("D", [256, 128], ids=["d256", "d128"])
@pytest.mark.parametrize("bk,bv", BODIES, ids=["%d/%ds" % b for b in BODIES])
def test_scalar_body_vs_oracle(oracle, lib, dev, bk, bv, D):
    """Two KV heads, an fp16 sink, 9 sealed groups, a tq6_0 tail of 301 positions; width 4 at GQA 4:1 (16 rows
    per KV head), then 5 positions x GQA 8 (40 rows: three tiles) whose causal ends fall inside the body."""
    H, S, G = 2, 128, 128
    ngr = 9
    B = S + ngr * G
    n_pos = B + 301
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, 0, 256, 512, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        K, V = inputs.kv_rows(n_pos, H, D, seed=700 + 10 * bk + bv + D)
        oracle_store(oracle, OL, K, V, 0)
        dK, dV = dev.put(K), dev.put(V)
        sjk.check(lib.sjk_hip_layer_store(C.byref(view), 0, n_pos, dK, dV, 1, None), "layer_store")
        oracle.layer_seal(C.byref(OL), S, B)
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, B, 16, None), "commit")
        dev.sync()
        body_b = ngr * H * OL.lay.bytes
        assert np.array_equal(dev.get(C.c_void_p(view.body), body_b, np.uint8), host_bytes(OL.body, body_b))
        rng = np.random.default_rng(bk * 10 + bv)
        for n_q, gq, qpos0 in ((4, 4, n_pos - 4), (5, 8, B - 300)):
            n_head = gq * H
            q = rng.standard_normal((n_q, n_head, D)).astype(np.float32)
            dq, do = dev.put(q), dev.alloc(q.nbytes)
            sjk.check(lib.sjk_hip_attend(C.byref(view), B, n_pos, qpos0, n_q, n_head, dq, 0.0625, do, None), "attend")
            got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
            rows = [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
            worst, l2 = check_rows(got, oracle_rows(oracle, OL, B, n_pos, q, qpos0, 0.0625, rows))
            say("[scalar] D=%d %d/%ds n_q=%d gq=%d qpos0=%d: worst %.4f of the tolerance, rel L2 %.2e" %
                (D, bk, bv, n_q, gq, qpos0, worst, l2))
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


@pytest.mark.parametrize("bk,bv,d,h", [(3, 3, 256, 4), (4, 2, 128, 8)], ids=["100k-d256-3/3s", "100k-d128-h8-4/2s"])
def test_scalar_body_100k_vs_oracle(oracle, lib, dev, bk, bv, d, h):
    """N = 100,000 through the default decode schedule (B = 94,336, tail 5,664, fp16 sink 128), width 4, GQA 4:1;
    sampled (row, head) pairs against the oracle's loop; repeated calls give the same bits."""
    N = 100000
    n_q, n_head = 4, 4 * h
    cfg, L, view, B, n_body, tail, _ = contexts.attention_context(lib, dev, None, N, bk, bv, 0, log=say, d=d, h=h,
                                                                  n_head=n_head)
    OL = None
    try:
        assert (B, n_body, tail) == (94336, 736, 5664)
        q = np.random.default_rng(4).standard_normal((n_q, n_head, d)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        scale = 1.0 / float(np.sqrt(d))
        sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, N - n_q, n_q, n_head, dq, scale, do, None), "attend")
        got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
        for rep in range(10):                     # the same bits on every call
            sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, N - n_q, n_q, n_head, dq, scale, do, None), "attend")
            again = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
            assert np.array_equal(again.view(np.uint32), got.view(np.uint32)), rep
        OL = contexts.oracle_layer_from_device(oracle, dev, cfg, L, n_body)
        rng = np.random.default_rng(bk + bv)
        pairs = [(0, 0), (n_q - 1, n_head - 1)] + [(int(a), int(b)) for a, b in zip(rng.integers(0, n_q, 6),
                                                                                    rng.integers(0, n_head, 6))]
        say("[scalar] oracle layer_attend_row for %d (row, head) pairs at N=100K, D=%d %d/%ds" % (len(pairs), d, bk, bv))
        worst, l2 = check_rows(got, oracle_rows(oracle, OL, B, N, q, N - n_q, scale, pairs))
        say("[scalar] 100K D=%d %d/%ds: worst %.4f of the tolerance, rel L2 %.2e" % (d, bk, bv, worst, l2))
    finally:
        if OL is not None:
            oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(L))
