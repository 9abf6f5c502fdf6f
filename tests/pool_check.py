"""Sampled oracle checks of a pool stress run (sj-kvarn-codec_amd/pool_stress.py): sealed records of a
(sequence, layer) re-sealed on the CPU from the same input rows, and decode attention of a (sequence,
layer) against the oracle's position-ordered loop over the same cache bytes. Test infrastructure: used by
tests/ and by bench.py's checker leg only."""
import ctypes as C

import numpy as np

import cabi


def oracle_layer(orc, ps, s, il):
    """An oracle layer holding the device bytes of (sequence s, layer il): sink, ring, and the sealed
    records in group order (the device keeps them at the pool blocks of the sequence's block table)."""
    ocfg = cabi.Config.from_buffer_copy(bytes(ps.cfg))
    OL = cabi.Layer()
    if orc.layer_init(C.byref(OL), C.byref(ocfg)) != 0:
        raise RuntimeError("oracle layer_init failed")
    seq = ps.seqs[s]
    L = seq.layers[il]
    H, D, S, G = ps.H, ps.D, ps.S, ps.G
    for name, nb in (("sink", S * H * D * 4), ("ring", L.cap * H * 2 * L.stage_bytes)):
        b = ps.dev.get(C.c_void_p(getattr(L, name)), nb, np.uint8)
        C.memmove(getattr(OL, name), b.ctypes.data, nb)
    rb = H * L.lay.bytes
    for g in range((seq.pol.B - S) // G):
        b = ps.dev.get(C.c_void_p(L.body + seq.blocks[g] * rb), rb, np.uint8)
        C.memmove(C.cast(OL.body, C.c_void_p).value + g * rb, b.ctypes.data, rb)
    return OL


def check_records(orc, ps, s, il, groups):
    """Re-seal groups of (s, il) on the CPU from the rows the run stored; returns the number of records
    (group x head) that are byte-identical to the device's."""
    ocfg = cabi.Config.from_buffer_copy(bytes(ps.cfg))
    seq = ps.seqs[s]
    L = seq.layers[il]
    H, S, G = ps.H, ps.S, ps.G
    rb = L.lay.bytes
    equal = 0
    for g in groups:
        OL = cabi.Layer()
        assert orc.layer_init(C.byref(OL), C.byref(ocfg)) == 0
        try:
            p0 = S + g * G
            K, V = ps.rows(s, il, p0, G)
            for i in range(G):
                kr, vr = K[i].copy(), V[i].copy()
                orc.rotate_heads(cabi.ptr(kr, cabi.f32p), H, ps.D)
                orc.rotate_heads(cabi.ptr(vr, cabi.f32p), H, ps.D)
                orc.layer_store(C.byref(OL), p0 + i, cabi.ptr(kr, cabi.f32p), cabi.ptr(vr, cabi.f32p))
            orc.layer_seal(C.byref(OL), p0, p0 + G)
            want = np.ctypeslib.as_array(C.cast(C.cast(OL.body, C.c_void_p).value + g * H * rb,
                                                C.POINTER(C.c_uint8)), shape=(H * rb,)).copy()
            got = ps.dev.get(C.c_void_p(L.body + seq.blocks[g] * H * rb), H * rb, np.uint8)
            equal += sum(int(np.array_equal(got[h * rb:(h + 1) * rb], want[h * rb:(h + 1) * rb])) for h in range(H))
        finally:
            orc.layer_free(C.byref(OL))
    return equal


def check_attention(orc, ps, s, il, rows):
    """Device decode attention of (s, il) for its last `width` positions vs the oracle's loop; returns the
    worst error / (1e-3 + 1e-3 |want|) over the sampled (row, head) pairs."""
    out = ps.dout[s]
    ps.attend(s, il, out)
    q = ps.q[s]
    got = ps.dev.get(out, q.nbytes, np.float32).reshape(q.shape)
    OL = oracle_layer(orc, ps, s, il)
    seq = ps.seqs[s]
    worst = 0.0
    try:
        gq = ps.n_head // ps.H
        for iq, hq in rows:
            want = np.zeros(ps.D, np.float32)
            qq = np.ascontiguousarray(q[iq, hq])
            orc.layer_attend_row(C.byref(OL), seq.pol.B, seq.n, cabi.ptr(qq, cabi.f32p), hq // gq,
                                 seq.n - ps.width + iq, ps.scale, cabi.ptr(want, cabi.f32p))
            worst = max(worst, float(np.max(np.abs(got[iq, hq] - want) / (1e-3 + 1e-3 * np.abs(want)))))
    finally:
        orc.layer_free(C.byref(OL))
    return worst
