"""The C ABI of libsjk.so on the CPU (no GPU calls): the library loads, exports every function that
include/sjk.h declares, and its host-side integer logic (record layout, payload order, journal policy,
ring slots, status strings, fp16 helpers) agrees with the oracle everywhere it is exercised."""
import ctypes as C
import os
import re
import sys

import numpy as np
import pytest

import cabi

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

HEADER = os.path.join(cabi.ROOT, "include", "sjk.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(sjk.LIB_PATH):
        pytest.fail("libsjk.so is not built: run __graft_entry__.build()")
    return sjk.load()


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    names = set(re.findall(r"\b((?:sj_kvarn|sjk)_\w+)\s*\(", text))
    types = {"sj_kvarn_body", "sj_kvarn_staging", "sj_kvarn_sink_type"}
    return sorted(n for n in names if n not in types)


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 70
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(sjk.SIGNATURES), set(names) ^ set(sjk.SIGNATURES)


def test_layout_and_payload_order_match_oracle(oracle, lib):
    for D in (32, 64, 128, 256, 512):
        for G in (16, 64, 128):
            for bk in (2, 3, 4):
                for bv in (2, 3, 4):
                    for body in (0, 1):
                        lo, lp = cabi.Layout(), sjk.Layout()
                        ro = oracle.layout_init(C.byref(lo), D, G, bk, bv, body)
                        rp = lib.sj_kvarn_layout_init(C.byref(lp), D, G, bk, bv, body)
                        assert ro == rp
                        if ro:
                            continue
                        assert bytes(lo) == bytes(lp)
                        assert oracle.record_bytes(D, G, bk, bv) == lib.sj_kvarn_record_bytes(D, G, bk, bv)
                        if D == 256 and G == 128:
                            for d in range(0, D, 3):
                                assert oracle.k_ch_idx(C.byref(lo), d) == lib.sj_kvarn_k_ch_idx(C.byref(lp), d)
                                assert oracle.v_ch_idx(C.byref(lo), d) == lib.sj_kvarn_v_ch_idx(C.byref(lp), d)
                                for t in range(0, G, 5):
                                    for v in (0, 1):
                                        assert oracle.code_bit(C.byref(lo), t, d, v) == \
                                            lib.sj_kvarn_code_bit(C.byref(lp), t, d, v)
    for b in (0, 1, 2):
        for bk in (2, 3, 4):
            for bv in (2, 3, 4):
                assert oracle.body_resolve(b, bk, bv) == lib.sj_kvarn_body_resolve(b, bk, bv)


def test_workspace_figure_matches_reference_abi(oracle, lib):
    for D in (128, 256):
        lo = oracle.layout(D, 128, 4, 4, 0)
        lp = sjk.Layout.from_buffer_copy(bytes(lo))
        assert oracle.seal_workspace_bytes(C.byref(lo)) == lib.sj_kvarn_seal_workspace_bytes(C.byref(lp))


def test_policy_schedule_matches_oracle(oracle, lib):
    rng = np.random.default_rng(4)
    for tail, tail_max, flush in ((4096, 8192, 0), (256, 512, 1), (256, 0, 0), (384, 640, 2)):
        po, pp = cabi.Policy(), sjk.Policy()
        oracle.policy_init(C.byref(po), 128, tail, tail_max, 128, flush)
        lib.sj_kvarn_policy_init(C.byref(pp), 128, tail, tail_max, 128, flush)
        pos = 0
        for step in range(3000):
            r = rng.random()
            if r < 0.05:
                n = int(rng.integers(1, 512))
            else:
                n = int(rng.integers(1, 5))
            if r > 0.995 and po.B_pending == po.B:
                cut = int(rng.integers(0, pos + 1))
                a = oracle.policy_truncate(C.byref(po), cut, None)
                b = lib.sj_kvarn_policy_truncate(C.byref(pp), cut, None)
                assert a == b
                pos = min(pos, a) if a != 0xFFFFFFFF else pos
            elif r > 0.98:
                keep = int(rng.integers(0, 9000))
                a = oracle.policy_idle(C.byref(po), pos, keep)
                b = lib.sj_kvarn_policy_idle(C.byref(pp), pos, keep)
                assert a == b
                oracle.policy_commit(C.byref(po))
                lib.sj_kvarn_policy_commit(C.byref(pp))
            else:
                a = oracle.policy_begin_ubatch(C.byref(po), pos, n)
                b = lib.sj_kvarn_policy_begin_ubatch(C.byref(pp), pos, n)
                assert a == b
                oracle.policy_commit(C.byref(po))
                lib.sj_kvarn_policy_commit(C.byref(pp))
                pos += n
            assert bytes(po) == bytes(pp), step
        for p in range(0, 20000, 37):
            assert oracle.group_floor(128, 128, p) == lib.sj_kvarn_group_floor(128, 128, p)
            assert oracle.policy_trunc_floor(C.byref(po), p) == lib.sj_kvarn_policy_trunc_floor(C.byref(pp), p)
            assert oracle.ring_slot(128, 9344, p + 128) == lib.sj_kvarn_ring_slot(128, 9344, p + 128)
    for args in ((4096, 8192, 128, 512), (256, 512, 128, 64), (4096, 0, 128, 1)):
        assert oracle.ring_capacity(*args) == lib.sj_kvarn_ring_capacity(*args)


def test_policy_idle_matches_oracle(oracle, lib):
    for keep in (0, 100, 4096, 5000, 20000):
        for end in range(0, 30000, 977):
            po, pp = cabi.Policy(), sjk.Policy()
            oracle.policy_init(C.byref(po), 128, 4096, 8192, 128, 0)
            lib.sj_kvarn_policy_init(C.byref(pp), 128, 4096, 8192, 128, 0)
            assert oracle.policy_idle(C.byref(po), end, keep) == lib.sj_kvarn_policy_idle(C.byref(pp), end, keep)
            assert bytes(po) == bytes(pp)


def test_config_strerror_fp16_helpers(oracle, lib):
    assert bytes(oracle.config_default(256, 4, 100000, 512)) == bytes(lib.sj_kvarn_config_default(256, 4, 100000, 512))
    for code in list(range(-11, 1)) + list(range(-131, -99)):
        a, b = oracle.strerror(code), lib.sj_kvarn_strerror(code)
        if a != b"unknown SJ-KVaRN status code":
            assert a == b, code
    assert b"HIP" in lib.sj_kvarn_strerror(-140)
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00001, 0x477FEFFF, 0x477FF000,
                                     0x33000000, 0x33000001, 0x387FE000], np.uint32)])
    for w in bits[::97].tolist() + bits[-10:].tolist():
        f = C.c_float(np.array([w], np.uint32).view(np.float32)[0])
        assert oracle.f32_to_f16(f) == lib.sj_kvarn_f32_to_f16(f)
    for h in range(0, 65536, 7):
        a, b = oracle.f16_to_f32(h), lib.sj_kvarn_f16_to_f32(h)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32) or (a != a and b != b)


def test_attend_rejects_a_tail_without_a_ring(lib):
    """A view whose visible positions reach past the sealed body must carry a ring of >= 16 slots: the
    attention kernels read the tail in 16-position chunks with one wrap at most (layers built by
    sj_kvarn_layer_init have >= 128 slots, sj_kvarn.h:1400-1403). The check is on the host: no GPU call."""
    v = sjk.View()
    assert lib.sj_kvarn_layout_init(C.byref(v.lay), 256, 128, 4, 4, 0) == 0
    v.n_head_kv, v.S, v.stage_bytes = 4, 128, 196
    fake = C.c_void_p(0x1000)                    # never dereferenced: the call is refused first
    v.sink, v.body = fake, fake
    v.work, v.work_bytes = fake, 1 << 30
    B = 128 + 4 * 128
    for ring, cap in ((None, 0), (fake, 0), (fake, 8), (fake, 15)):
        v.ring, v.cap = ring, cap
        assert lib.sjk_hip_attend(C.byref(v), B, B + 10, B + 6, 4, 16, fake, 0.0625, fake, None) == -100, (ring, cap)
        job = sjk.AttendJob(v, B, B + 10, B + 6, fake, fake)
        assert lib.sjk_hip_attend_batch(C.byref(job), 1, 4, 16, 0.0625, None) == -100


def test_attend_dyn_checks_its_arguments_on_the_host(lib):
    """sjk_hip_attend_dyn refuses missing pointers and a query head count that is not a multiple of the KV
    heads before any GPU call; the context itself is checked on the device, from the descriptor."""
    v = sjk.View()
    assert lib.sj_kvarn_layout_init(C.byref(v.lay), 256, 128, 4, 4, 0) == 0
    v.n_head_kv, v.S, v.stage_bytes = 4, 128, 196
    fake = C.c_void_p(0x1000)                    # never dereferenced: the call is refused first
    v.sink, v.body, v.ring, v.cap = fake, fake, fake, 256
    v.work, v.work_bytes = fake, 1 << 30
    for desc, q, out, n_q, n_head in ((None, fake, fake, 4, 16), (fake, None, fake, 4, 16), (fake, fake, None, 4, 16),
                                      (fake, fake, fake, 0, 16), (fake, fake, fake, 4, 6), (fake, fake, fake, 4, 0)):
        assert lib.sjk_hip_attend_dyn(C.byref(v), desc, 4096, n_q, n_head, q, 0.0625, out, None) == -100
    assert lib.sjk_hip_attend_dyn(None, fake, 4096, 4, 16, fake, 0.0625, fake, None) == -100


def test_attend_needs_a_workspace(lib):
    """The attention calls keep their partial results in the view's workspace (sjk_hip_view.work, which
    sjk_layer_view fills with the layer's own): a view without one is refused on the host, before any GPU call.
    sjk_hip_workspace_bytes sizes one for a hand-built view."""
    v = sjk.View()
    assert lib.sj_kvarn_layout_init(C.byref(v.lay), 256, 128, 4, 4, 0) == 0
    v.n_head_kv, v.S, v.stage_bytes = 4, 128, 196
    fake = C.c_void_p(0x1000)
    v.sink, v.body, v.ring, v.cap = fake, fake, fake, 256
    assert lib.sjk_hip_attend(C.byref(v), 256, 300, 296, 4, 16, fake, 0.0625, fake, None) == -100
    job = sjk.AttendJob(v, 256, 300, 296, fake, fake)
    assert lib.sjk_hip_attend_batch(C.byref(job), 1, 4, 16, 0.0625, None) == -100
    assert lib.sjk_hip_workspace_bytes(C.byref(v.lay), 4) > 16 * 258 * 4 * 256
    assert lib.sjk_hip_workspace_bytes(C.byref(v.lay), 0) == 0


def test_attend_refuses_views_outside_the_kernels(lib):
    """A hand-built view that no layer can have (group 64, or a record layout with its blocks in another order) is
    refused by every attention entry point with SJK_ERR_UNSUPPORTED and a message, before any GPU call; the same
    view with a layer's own layout passes these checks (it is refused only later, for its missing workspace)."""
    fake = C.c_void_p(0x1000)                    # never dereferenced: the call is refused first

    def view(G, swap=False):
        v = sjk.View()
        assert lib.sj_kvarn_layout_init(C.byref(v.lay), 256, G, 4, 4, 0) == 0
        if swap:                                 # the V payload before the K payload
            v.lay.k_payload, v.lay.v_payload = v.lay.v_payload, v.lay.k_payload
        v.n_head_kv, v.S, v.stage_bytes = 4, 128, 196
        v.sink, v.body, v.ring, v.cap = fake, fake, fake, 256
        v.work, v.work_bytes = fake, 1 << 30
        return v

    for v in (view(64), view(128, swap=True)):
        assert lib.sjk_hip_attend(C.byref(v), 256, 300, 296, 4, 16, fake, 0.0625, fake, None) == -141
        assert b"not one the attention kernels are built for" in lib.sjk_last_error()
        job = sjk.AttendJob(v, 256, 300, 296, fake, fake)
        assert lib.sjk_hip_attend_batch(C.byref(job), 1, 4, 16, 0.0625, None) == -141
        assert lib.sjk_hip_attend_noalloc(C.byref(v), 256, 300, 296, 4, 16, fake, 0.0625, fake, None) == -141
        assert lib.sjk_hip_attend_dyn(C.byref(v), fake, 4096, 4, 16, fake, 0.0625, fake, None) == -141
        assert b"sjk_hip_attend_dyn" in lib.sjk_last_error()
    v = view(128)
    v.work = None
    assert lib.sjk_hip_attend(C.byref(v), 256, 300, 296, 4, 16, fake, 0.0625, fake, None) == -100


def test_head_dim_beyond_the_kernels_is_refused_with_a_status(oracle, lib):
    """A layer of head_dim 512 (a multiple of 128 that the reference accepts, sj_kvarn.h:1447-1449) is refused at
    creation with SJK_ERR_UNSUPPORTED and a message, before any device allocation, instead of aborting; the
    reference's own argument checks come first (head_dim 96 is no multiple of 128: its -10)."""
    for D, want in ((512, -141), (96, -10)):
        cfg = lib.sj_kvarn_config_default(D, 4, 4096, 64)
        L = sjk.Layer()
        assert lib.sj_kvarn_layer_init(C.byref(L), C.byref(cfg)) == want, D
        assert lib.sj_kvarn_strerror(want)
    assert b"head_dim 128/256" in lib.sj_kvarn_strerror(-141)
    ocfg = oracle.config_default(512, 4, 4096, 64)
    OL = cabi.Layer()
    assert oracle.layer_init(C.byref(OL), C.byref(ocfg)) == 0     # the reference's rules accept it
    oracle.layer_free(C.byref(OL))


def test_seal_group_aborts_on_a_layout_the_device_seal_lacks():
    """sj_kvarn_seal_group is void (sj_kvarn.h:203-204): a layout the HIP seal is not built for (D = 512, or a scalar
    group of 64, which the reference seals) cannot return a status, and a record left unwritten would pass for a
    sealed one, so the call aborts with a message naming the layout (before any GPU call), as the library's other
    void calls do on a device failure."""
    import subprocess
    code = (
        "import ctypes as C, sys; sys.path.insert(0, %r); import sjk; lib = sjk.load(); lay = sjk.Layout()\n"
        "D, G = %%d, %%d\n"
        "assert lib.sj_kvarn_layout_init(C.byref(lay), D, G, 4, 4, 0) == 0\n"
        "K = (C.c_uint16 * (D * G))(); V = (C.c_uint16 * (D * G))(); rec = (C.c_uint8 * lay.bytes)()\n"
        "lib.sj_kvarn_seal_group(C.byref(lay), K, V, D, 16, rec, None)\n"
        "print('RETURNED')\n" % cabi.PKG)
    for D, G in ((512, 128), (256, 64)):
        out = subprocess.run([sys.executable, "-c", code % (D, G)], capture_output=True, text=True, timeout=120)
        assert out.returncode != 0 and "RETURNED" not in out.stdout, (D, G, out.stdout, out.stderr[-500:])
        assert "sj_kvarn_seal_group" in out.stderr and "D=%d G=%d" % (D, G) in out.stderr, out.stderr[-500:]
