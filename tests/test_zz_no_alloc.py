"""sjk_hip_attend_noalloc: the attention entry point that allocates nothing (its partial results go to a static
device array instead of the view's workspace). Two calls in a row, the second with a smaller input (fewer query
rows over a shorter context), each bit-equal to sjk_hip_attend's output on the same view with its own workspace;
the 4/4 matrix-core kernel at D = 256 and 128, the other scalar bodies' kernel (4/2 at D = 128) and the trellis
kernel (3/3 at D = 128). A view whose workspace would exceed the static array is refused on the host."""
import ctypes as C
import sys

import numpy as np
import pytest

import cabi

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

from test_gpu_layer import device_context, make_pair  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.fixture(scope="module")
def dev():
    d = sjk.Device()
    yield d
    d.free_all()


@pytest.mark.parametrize("D,H,bk,bv,body", [(256, 4, 4, 4, 0), (128, 2, 4, 4, 0), (128, 2, 4, 2, 0), (128, 2, 3, 3, 1)],
                         ids=["4/4-d256", "4/4-d128", "4/2-d128", "3/3t-d128"])
def test_noalloc_matches_attend(oracle, lib, dev, D, H, bk, bv, body):
    S, G = 128, 128
    B = S + 40 * G
    n_pos = B + 700
    OL, PL = make_pair(oracle, lib, D, H, bk, bv, body, 256, 1024, n_ctx=n_pos + 64, n_ubatch=512)
    view = lib.sjk_layer_view(C.byref(PL))
    try:
        device_context(oracle, lib, dev, OL, PL, view, n_pos, B, seed=8100 + D)
        bare = sjk.View.from_buffer_copy(bytes(view))
        bare.work, bare.work_bytes = None, 0                      # no workspace: only the no-alloc entry takes it
        rng = np.random.default_rng(3)
        free_b, total_b = C.c_size_t(0), C.c_size_t(0)
        dev.hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]

        def free_bytes():
            dev.sync()
            dev._ck(dev.hip.hipMemGetInfo(C.byref(free_b), C.byref(total_b)), "hipMemGetInfo")
            return free_b.value

        # second call: a smaller input (one position, 4 query heads, an earlier causal end)
        for k, (n_q, n_head, N, qpos0) in enumerate(((4, 4 * H, n_pos, n_pos - 4), (1, H, B + 100, B + 50))):
            q = rng.standard_normal((n_q, n_head, D)).astype(np.float32)
            dq, d1, d2 = dev.put(q), dev.alloc(q.nbytes), dev.alloc(q.nbytes)
            before = free_bytes()
            sjk.check(lib.sjk_hip_attend_noalloc(C.byref(bare), B, N, qpos0, n_q, n_head, dq, 0.0625, d1, None),
                      "sjk_hip_attend_noalloc")
            if k:                  # the call allocates no device memory (the first call may load code objects)
                assert free_bytes() == before
            sjk.check(lib.sjk_hip_attend(C.byref(view), B, N, qpos0, n_q, n_head, dq, 0.0625, d2, None), "sjk_hip_attend")
            a = dev.get(d1, q.nbytes, np.uint32)
            b = dev.get(d2, q.nbytes, np.uint32)
            assert np.array_equal(a, b), (n_q, n_head, N)
            assert np.all(np.isfinite(a.view(np.float32)))
            assert lib.sjk_hip_attend(C.byref(bare), B, N, qpos0, n_q, n_head, dq, 0.0625, d2, None) == -100
    finally:
        oracle.layer_free(C.byref(OL))
        lib.sj_kvarn_layer_free(C.byref(PL))


def test_noalloc_refuses_views_beyond_the_scratch(lib):
    """64 KV heads at D = 256 need more partial slots than the 16 MiB array holds: refused before any launch."""
    v = sjk.View()
    assert lib.sj_kvarn_layout_init(C.byref(v.lay), 256, 128, 4, 4, 0) == 0
    v.n_head_kv, v.S, v.stage_bytes = 64, 128, 196
    fake = C.c_void_p(0x1000)                    # never dereferenced: the call is refused first
    v.sink, v.body, v.ring, v.cap = fake, fake, fake, 256
    assert lib.sjk_hip_workspace_bytes(C.byref(v.lay), 64) > 16 << 20
    assert lib.sjk_hip_attend_noalloc(C.byref(v), 256, 300, 296, 1, 64, fake, 0.0625, fake, None) == -109
    assert b"16 MiB" in lib.sjk_last_error()
