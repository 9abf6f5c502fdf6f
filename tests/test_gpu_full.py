"""Parity at the BASELINE configs' full sizes, and the two numeric assumptions of the device seal.

  * the whole 4096-token commit (32 groups x 4 KV heads = 128 records, 4/4 scalar and
    3/2 trellis) sealed straight out of the device ring; the ring must equal the oracle's own store of the same
    rows and every record must equal the oracle's layer_seal of that ring, byte for byte.
  * N = 100,000 through the default decode schedule (B = 94,336, tail 5,664, fp16 sink 128),
    width 4, 16 query heads on 4 KV heads; sampled (row, head) pairs against the oracle's loop within
    max-abs 1e-3 + rel 1e-3 (4/4 and the trellis bodies), and the same context at head dimension 128 with
    8 KV heads and 32 query heads (the 4/4 matrix-core kernel at D = 128).
  * the whole per-sequence stress (16 layers x 8 sequences x 2048 decode rounds, 3/3 trellis, with
    the truncation and the state save / restore); sampled records re-sealed by the oracle from the run's input
    rows, sampled attention rows against the oracle's loop.
  * fp16: every one of the 2^32 float bit patterns through the device's F16 staging (f32 -> f16 of
    sj_kvarn.h:693-711), against the hardware's round-to-nearest-even cast with the reference's NaN rule (and
    numpy's cast on the half range).
  * libm: the balance's log-domain scale update (sj_kvarn.h:1000-1002) with the device's log / exp against
    the host libm the reference calls (the oracle, gcc + glibc).
"""
import ctypes as C
import os
import sys
import threading
import time

import numpy as np
import pytest

import cabi
import contexts
import inputs
import pool_check

sys.path.insert(0, cabi.PKG)
import pool_stress  # noqa: E402
import sjk  # noqa: E402

pytestmark = pytest.mark.gpu
ATOL = RTOL = 1e-3
S, G, H, D = contexts.S, contexts.G, contexts.H, contexts.D
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


def parallel(fn, items, n_threads=N_THREADS):
    """fn(item) over items on host threads (the oracle's ctypes calls release the GIL)"""
    out = {}

    def work(k):
        for it in items[k::n_threads]:
            out[it] = fn(it)

    ths = [threading.Thread(target=work, args=(k,)) for k in range(n_threads)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    return out


@pytest.mark.parametrize("bk,bv,body", [(4, 4, 0), (3, 2, 1)], ids=["configs1-4/4s", "configs2-3/2t"])
def test_full_commit_vs_oracle(oracle, lib, dev, bk, bv, body):
    say("[full] commit %d/%d%s: store %d positions on the device" % (bk, bv, "t" if body else "s", S + contexts.TAIL_MAX))
    cfg, L, view, K, V = contexts.commit_ring(lib, dev, None, bk, bv, body)
    OL = None
    layers = []
    try:
        # the oracle's own store of the same rows (engine order: rotate every head, then store)
        ocfg = cabi.Config.from_buffer_copy(bytes(cfg))
        OL = cabi.Layer()
        assert oracle.layer_init(C.byref(OL), C.byref(ocfg)) == 0
        for p in range(K.shape[0]):
            kr, vr = K[p].copy(), V[p].copy()
            oracle.rotate_heads(cabi.ptr(kr, cabi.f32p), H, D)
            oracle.rotate_heads(cabi.ptr(vr, cabi.f32p), H, D)
            oracle.layer_store(C.byref(OL), p, cabi.ptr(kr, cabi.f32p), cabi.ptr(vr, cabi.f32p))
        ring_b = L.cap * H * 2 * L.stage_bytes
        assert np.array_equal(dev.get(C.c_void_p(L.ring), ring_b, np.uint8),
                              np.ctypeslib.as_array(C.cast(OL.ring, cabi.u8p), shape=(ring_b,)))
        sink_b = S * H * D * 4
        assert np.array_equal(dev.get(C.c_void_p(L.sink), sink_b, np.uint8),
                              np.ctypeslib.as_array(C.cast(OL.sink, cabi.u8p), shape=(sink_b,)))
        say("[full] device commit of 4096 tokens (128 records)")
        sjk.check(lib.sjk_hip_commit(C.byref(view), 1, S, S + 4096, 16, None), "sjk_hip_commit")
        dev.sync()
        rb = L.lay.bytes
        got = dev.get(C.c_void_p(L.body), 32 * H * rb, np.uint8)
        # the oracle seals the same 32 groups from the same ring on host threads (one layer per thread)
        layers = [OL] + [contexts.oracle_layer_from_device(oracle, dev, cfg, L, 0) for _ in range(N_THREADS - 1)]
        say("[full] oracle layer_seal of the 32 groups on %d threads" % N_THREADS)
        t0 = time.perf_counter()
        owner = {g: g % N_THREADS for g in range(32)}

        def seal(g):
            ly = layers[owner[g]]
            oracle.layer_seal(C.byref(ly), S + g * G, S + (g + 1) * G)
            base = C.cast(ly.body, C.c_void_p).value + g * H * rb
            return np.ctypeslib.as_array(C.cast(base, cabi.u8p), shape=(H * rb,)).copy()

        want = parallel(seal, list(range(32)))
        say("[full] oracle done in %.1f s" % (time.perf_counter() - t0))
        bad = [(g, h) for g in range(32) for h in range(H)
               if not np.array_equal(got[(g * H + h) * rb:(g * H + h + 1) * rb], want[g][h * rb:(h + 1) * rb])]
        assert not bad, "records differing from the oracle: %s" % bad[:8]
    finally:
        for ly in layers:
            oracle.layer_free(C.byref(ly))
        if OL is not None and not layers:
            oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(L))


@pytest.mark.parametrize("bk,bv,body,n_pairs,d,h", [(4, 4, 0, 64, D, H), (3, 3, 1, 64, D, H), (3, 2, 1, 4, D, H),
                                                     (2, 2, 1, 4, D, H), (4, 4, 0, 16, 128, 8), (3, 3, 1, 4, 128, 8)],
                         ids=["configs3-4/4s", "100k-3/3t", "100k-3/2t", "100k-2/2t", "100k-d128-h8-4/4s",
                              "100k-d128-h8-3/3t"])
def test_attention_100k_vs_oracle(oracle, lib, dev, bk, bv, body, n_pairs, d, h):
    N = 100000
    n_q, n_head = 4, 4 * h                       # width 4, GQA 4:1
    cfg, L, view, B, n_body, tail, _ = contexts.attention_context(lib, dev, None, N, bk, bv, body, log=say, d=d, h=h,
                                                                  n_head=n_head)
    OL = None
    try:
        assert (B, n_body, tail) == (94336, 736, 5664)
        scale = 1.0 / float(np.sqrt(d))
        q = np.random.default_rng(4).standard_normal((n_q, n_head, d)).astype(np.float32)
        dq, do = dev.put(q), dev.alloc(q.nbytes)
        qpos0 = N - n_q
        sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, qpos0, n_q, n_head, dq, scale, do, None), "attend")
        got = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
        assert np.all(np.isfinite(got))
        # the same call again and again gives the same bits (a missing hazard wait state inside a kernel shows as
        # output that varies from run to run)
        for rep in range(20):
            sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, qpos0, n_q, n_head, dq, scale, do, None), "attend")
            again = dev.get(do, q.nbytes, np.float32).reshape(q.shape)
            assert np.array_equal(again.view(np.uint32), got.view(np.uint32)), rep
        OL = contexts.oracle_layer_from_device(oracle, dev, cfg, L, n_body)
        rng = np.random.default_rng(n_pairs)
        if n_pairs >= n_q * n_head:              # every (row, head) pair of the call
            pairs = [(iq, hq) for iq in range(n_q) for hq in range(n_head)]
        else:
            pairs = [(0, 0), (n_q - 1, n_head - 1)] + [(int(a), int(b)) for a, b in
                                                       zip(rng.integers(0, n_q, n_pairs - 2),
                                                           rng.integers(0, n_head, n_pairs - 2))]
        say("[full] oracle layer_attend_row for %d (row, head) pairs at N=100K, D=%d" % (len(pairs), d))

        def att(pair):
            iq, hq = pair
            o = np.zeros(d, np.float32)
            qq = np.ascontiguousarray(q[iq, hq])
            oracle.layer_attend_row(C.byref(OL), B, N, cabi.ptr(qq, cabi.f32p), hq // 4, qpos0 + iq, scale,
                                    cabi.ptr(o, cabi.f32p))
            return o

        want = parallel(att, pairs)
        worst = max(float(np.max(np.abs(got[p] - want[p]) / (ATOL + RTOL * np.abs(want[p])))) for p in pairs)
        say("[full] worst error / tolerance %.4f" % worst)
        assert worst <= 1.0
    finally:
        if OL is not None:
            oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(L))


def test_pool_stress_full_configs4(oracle, lib, dev):
    ps, rep = pool_stress.run(lib, dev, inputs.kv_rows, log=say)
    try:
        say("[full] %s" % {k: rep[k] for k in ("commits", "truncate", "save_restore", "device_ms_per_round")})
        assert ps.n_layers == 16 and ps.n_seq == 8 and rep["rounds"] == 2048
        assert rep["commits"] >= ps.n_seq
        assert rep["truncate"]["B_after"] < rep["truncate"]["B_before"]
        sr = rep["save_restore"]
        assert sr["stream_equal"] and sr["attention_equal"] and sr["async_save"]["stream_equal_sync"]
        assert sr["async_save"]["rounds_during"] >= 1 and sr["async_restore"]["rounds_during"] >= 1
        last = lambda s: (ps.seqs[s].pol.B - S) // G - 1  # noqa: E731
        recs = [(0, 0, last(0)), (1, 15, 0), (5, 7, last(5)), (7, 3, last(7) // 2)]
        for s, il, g in recs:
            assert pool_check.check_records(oracle, ps, s, il, [g]) == H, (s, il, g)
        for s, il in ((0, 0), (7, 15), (1, 15)):
            worst = pool_check.check_attention(oracle, ps, s, il, [(0, 0), (3, 15), (2, 7)])
            assert worst <= 1.0, (s, il, worst)
    finally:
        ps.free()


def test_fp16_all_floats_on_device(lib, dev):
    """f32 -> f16 (sj_kvarn.h:693-711) on the device for all 2^32 bit patterns: the F16 staging path stores the
    conversion of each value (rows of 512 values). Expected: the hardware's IEEE round-to-nearest-even cast (torch
    .half() on the same GPU, an independent routine: v_cvt_f16_f32) with NaN -> sign | 0x7E00 as in the reference;
    chunks of the half range are also compared with numpy's cast on the host."""
    import torch
    chunk = 1 << 28
    bad = 0
    for i in range((1 << 32) // chunk):
        say("[fp16] chunk %d of %d" % (i, (1 << 32) // chunk))
        bits = torch.arange(i * chunk, (i + 1) * chunk, dtype=torch.int64, device="cuda").to(torch.int32)
        x = bits.view(torch.float32)
        got = torch.empty(chunk, dtype=torch.int16, device="cuda")
        torch.cuda.synchronize()
        sjk.check(lib.sjk_hip_stage(1, C.c_void_p(x.data_ptr()), C.c_void_p(got.data_ptr()), 512, 1024, chunk // 512,
                                    None), "sjk_hip_stage")
        torch.cuda.synchronize()
        want = x.half().view(torch.int16)
        nanv = ((bits >> 16) & 0x8000) | 0x7E00
        want = torch.where(torch.isnan(x), nanv.to(torch.int16), want)
        bad += int((got != want).sum().item())
        if i in (3, 4):   # exponents 0x30 .. 0x4F: all finite halves, their rounding boundaries and overflow
            xs = x[::7].cpu().numpy()
            with np.errstate(over="ignore", invalid="ignore"):
                w2 = xs.astype(np.float16).view(np.uint16)
            w2 = np.where(np.isnan(xs), (xs.view(np.uint32) >> 16 & 0x8000) | 0x7E00, w2).astype(np.uint16)
            bad += int(np.count_nonzero(got[::7].cpu().numpy().view(np.uint16) != w2))
        del bits, x, got, want, nanv
    assert bad == 0


def test_balance_log_exp_vs_host_libm(oracle, lib, dev):
    """The seal's scale update acc = clamp(acc + log(clamp(sd)), -0.3, 10), scale = (float) exp(acc) with the
    device's double log / exp against the host glibc the reference calls. The stored scales are floats: they
    must agree on every sample. The double accumulator (which carries into later passes) is compared too, and
    its mismatch rate reported; a carried 1-ulp difference shows up in the chained sample as a scale flip."""
    rng = np.random.default_rng(12)
    n = 1 << 23
    sd = np.exp(rng.uniform(np.log(1e-4), np.log(1e4), n)).astype(np.float32)
    acc = rng.uniform(-0.3, 10.0, n)
    sd[:8] = [1e-3, 1e3, 0.0, 1.0, np.float32(np.exp(-0.3)), 1e-3 * 0.99, 2e3, np.float32(np.exp(10.0))]
    acc[:8] = [0.0, 10.0, -0.3, 0.0, 0.0, -0.3, 9.0, 0.0]
    d_sd, d_acc, d_sc = dev.put(sd), dev.put(acc), dev.alloc(n * 4)
    sjk.check(lib.sjk_hip_balance_step(d_sd, d_acc, d_sc, n, None), "balance_step")
    g_acc, g_sc = dev.get(d_acc, n * 8, np.float64), dev.get(d_sc, n * 4, np.float32)
    w_acc, w_sc = acc.copy(), np.zeros(n, np.float32)
    oracle.balance_step(cabi.ptr(sd, cabi.f32p), w_acc.ctypes.data_as(C.POINTER(C.c_double)),
                        cabi.ptr(w_sc, cabi.f32p), n)
    acc_diff = int(np.count_nonzero(g_acc.view(np.uint64) != w_acc.view(np.uint64)))
    sc_diff = int(np.count_nonzero(g_sc.view(np.uint32) != w_sc.view(np.uint32)))
    say("[libm] %d samples: accumulator differs in %d (%.2e), scale in %d" % (n, acc_diff, acc_diff / n, sc_diff))
    assert sc_diff == 0
    # chains as in a seal: 32 passes carried through the same accumulator (the balance's 2 x 16 updates)
    m, steps = 1 << 18, 32
    a_dev = np.zeros(m)
    a_host = np.zeros(m)
    d_a = dev.put(a_dev)
    flips = 0
    for k in range(steps):
        s = np.exp(rng.normal(0.0, 1.5, m)).astype(np.float32)
        dev.upload(d_sd, s)
        sjk.check(lib.sjk_hip_balance_step(d_sd, d_a, d_sc, m, None), "balance_step")
        gs = dev.get(d_sc, m * 4, np.float32)
        ws = np.zeros(m, np.float32)
        oracle.balance_step(cabi.ptr(s, cabi.f32p), a_host.ctypes.data_as(C.POINTER(C.c_double)),
                            cabi.ptr(ws, cabi.f32p), m)
        flips += int(np.count_nonzero(gs.view(np.uint32) != ws.view(np.uint32)))
    a_dev = dev.get(d_a, m * 8, np.float64)
    say("[libm] chained: %d x %d steps, scale flips %d, final accumulators differing %d" %
        (m, steps, flips, int(np.count_nonzero(a_dev.view(np.uint64) != a_host.view(np.uint64)))))
    assert flips == 0
