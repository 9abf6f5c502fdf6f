"""Device caches at the BASELINE shapes, built through the product path (shared by the -m gpu tests and
bench.py): a layer's staging ring for the configs[1]/[2] commits, and the configs[3] decode-schedule
context of N positions (fp16 sink, sealed body up to B, tq6_0 tail).

Everything is stored with sjk_hip_layer_store (fused Hadamard + tq6_0) and sealed with sjk_hip_commit;
the inputs are tests/inputs.py's seeded rows, so a checker can rebuild any stored row.
"""
import ctypes as C
import sys

import numpy as np

import cabi
import inputs

sys.path.insert(0, cabi.PKG)
import sjk  # noqa: E402

D, H, S, G = 256, 4, 128, 128
TAIL, TAIL_MAX = 4096, 8192


def make_layer(lib, n_ctx, n_ubatch, bk=4, bv=4, body=0, d=D, h=H):
    cfg = lib.sj_kvarn_config_default(d, h, n_ctx, n_ubatch)
    cfg.bits_k, cfg.bits_v, cfg.body = bk, bv, body
    L = sjk.Layer()
    sjk.check(lib.sj_kvarn_layer_init(C.byref(L), C.byref(cfg)), "sj_kvarn_layer_init")
    return cfg, L


def store(lib, dev, view, K, V, pos0, stream):
    """append rows [pos0, pos0 + n) through the device path (rotation fused), synchronously"""
    dK, dV = dev.put(K), dev.put(V)
    sjk.check(lib.sjk_hip_layer_store(C.byref(view), pos0, K.shape[0], dK, dV, 1, stream), "layer_store")
    dev.hip.hipStreamSynchronize(stream)
    dev.free(dK)
    dev.free(dV)


def commit_ring(lib, dev, stream, bk, bv, body, seed=2024):
    """a layer whose ring holds S + TAIL_MAX stored positions, ready for the
    4096-token commit [S, S + 4096). Returns (cfg, layer, view, K, V) with the unrotated input rows."""
    cfg, L = make_layer(lib, n_ctx=16384, n_ubatch=512, bk=bk, bv=bv, body=body)
    view = lib.sjk_layer_view(C.byref(L))
    K, V = inputs.kv_rows(S + TAIL_MAX, H, D, seed=seed)
    store(lib, dev, view, K, V, 0, stream)
    return cfg, L, view, K, V


def decode_schedule_B(lib, N):
    """sealed end B after decoding to N one token at a time under the default policy, and the commits
    (pos0, B_from, B_to) on the way"""
    pol = sjk.Policy()
    lib.sj_kvarn_policy_init(C.byref(pol), S, TAIL, TAIL_MAX, G, 0)
    commits = []
    p = S + TAIL + 1
    while True:
        # the next commit happens at the first pos0 with pos0 - B >= tail_max
        pos0 = max(p, pol.B + TAIL_MAX)
        if pos0 >= N:
            break
        lib.sj_kvarn_policy_begin_ubatch(C.byref(pol), pos0, 1)
        if pol.B_pending > pol.B:
            commits.append((pos0, pol.B, pol.B_pending))
        lib.sj_kvarn_policy_commit(C.byref(pol))
        p = pos0 + 1
    return pol.B, commits


def attention_context(lib, dev, stream, N, bk=4, bv=4, body=0, seed=7000, log=None, d=D, h=H, n_head=16):
    """a decode-schedule context of N positions built through the product path (head dimension d,
    h KV heads; configs[3] is d = 256, h = 4). Returns (cfg, layer, view, B, n_body, tail, algorithmic bytes
    of one width-4 call with n_head query heads)."""
    B, commits = decode_schedule_B(lib, N)
    if log:
        log("[ctx] building a %d-position context, D=%d, %d KV heads, body %d/%d%s (B=%d, %d commits on the way)" %
            (N, d, h, bk, bv, "t" if body else "", B, len(commits)))
    cfg, L = make_layer(lib, n_ctx=N + 1024, n_ubatch=1, bk=bk, bv=bv, body=body, d=d, h=h)
    v0 = lib.sjk_layer_view(C.byref(L))
    stored, Bcur = 0, S
    for (pos0, bfrom, bto) in commits + [(N, None, None)]:
        while stored < pos0:
            n = min(4096, pos0 - stored)
            Kc, Vc = inputs.kv_rows(n, h, d, seed=seed + stored)
            store(lib, dev, v0, Kc, Vc, stored, stream)
            stored += n
        if bfrom is not None:
            sjk.check(lib.sjk_hip_commit(C.byref(v0), 1, bfrom, bto, 16, stream), "commit")
            Bcur = bto
    dev.hip.hipStreamSynchronize(stream)
    assert Bcur == B
    n_body = (B - S) // G
    tail = N - B
    alg_bytes = n_body * h * L.lay.bytes + tail * h * 2 * L.stage_bytes + S * h * d * 4 + 4 * n_head * d * 2 + \
        4 * n_head * d * 4
    return cfg, L, v0, B, n_body, tail, alg_bytes


def oracle_layer_from_device(orc, dev, cfg, L, n_body_groups):
    """An oracle layer holding the same sink / ring / body bytes as a device layer (contiguous body)."""
    ocfg = cabi.Config.from_buffer_copy(bytes(cfg))
    OL = cabi.Layer()
    if orc.layer_init(C.byref(OL), C.byref(ocfg)) != 0:
        raise RuntimeError("oracle layer_init failed")
    d, h = cfg.head_dim, cfg.n_head_kv
    for name, n in (("ring", L.cap * h * 2 * L.stage_bytes), ("sink", S * h * d * 4),
                    ("body", n_body_groups * h * L.lay.bytes)):
        if n:
            b = dev.get(C.c_void_p(getattr(L, name)), n, np.uint8)
            C.memmove(getattr(OL, name), b.ctypes.data, n)
    return OL
