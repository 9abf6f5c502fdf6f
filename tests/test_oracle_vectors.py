"""The oracle against the reference's own known-answer vectors.

tests/golden/expected_vectors.txt is the reference's fixture (FNV-1a 64 of the records, decoded rows and
tq6_0 bytes produced by the llamAmpere tree encoder on the integer-only inputs of the reference's
tests/vector_inputs.h). The hashing protocol follows tests/test_vectors.c:20-70: record hash, then one
running hash over decode_k_row(t), decode_v_row(t) for t = 0..127.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

import cabi

GOLD = os.path.join(os.path.dirname(__file__), "golden", "expected_vectors.txt")
FNV0 = 1469598103934665603


def _lines():
    seal, tq6 = [], []
    for line in open(GOLD):
        m = re.match(r"seal D=(\d+) bk=(\d) bv=(\d) body=(\d) bytes=(\d+) rec=([0-9a-f]+) dec=([0-9a-f]+)", line)
        if m:
            seal.append(tuple(int(x) for x in m.groups()[:5]) + (int(m.group(6), 16), int(m.group(7), 16)))
        m = re.match(r"tq6 rows=(\d+) n=(\d+) enc=([0-9a-f]+) dec=([0-9a-f]+)", line)
        if m:
            tq6.append((int(m.group(1)), int(m.group(2)), int(m.group(3), 16), int(m.group(4), 16)))
    return seal, tq6


SEAL, TQ6 = _lines()


def test_fixture_complete():
    assert len(SEAL) == 20 and len(TQ6) == 1


@pytest.mark.parametrize("D,bk,bv,body,nbytes,erec,edec", SEAL, ids=["D%d-%d/%d-%s" % (s[0], s[1], s[2], "t" if s[3] else "s") for s in SEAL])
def test_seal_vector(oracle, D, bk, bv, body, nbytes, erec, edec):
    lay = oracle.layout(D, 128, bk, bv, body)
    assert lay.bytes == nbytes
    assert oracle.record_bytes(D, 128, bk, bv) == nbytes
    K = np.zeros(D * 128, np.uint16)
    V = np.zeros(D * 128, np.uint16)
    oracle.vec_fill_group(D, 128, 1, cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p))
    rec = np.zeros(lay.bytes, np.uint8)
    work = np.zeros(oracle.seal_workspace_bytes(C.byref(lay)), np.uint8)
    oracle.seal_group(C.byref(lay), cabi.ptr(K, cabi.u16p), cabi.ptr(V, cabi.u16p), D, 16, cabi.ptr(rec), work.ctypes.data_as(C.c_void_p))
    assert oracle.fnv1a(rec.ctypes.data, rec.nbytes, FNV0) == erec
    row = np.zeros(D, np.float32)
    h = FNV0
    for t in range(128):
        oracle.decode_k_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(row, cabi.f32p))
        h = oracle.fnv1a(row.ctypes.data, row.nbytes, h)
        oracle.decode_v_row(C.byref(lay), cabi.ptr(rec), t, cabi.ptr(row, cabi.f32p))
        h = oracle.fnv1a(row.ctypes.data, row.nbytes, h)
    assert h == edec


def test_tq6_vector(oracle):
    rows, n, eenc, edec = TQ6[0]
    x = np.zeros(rows * n, np.float32)
    oracle.vec_fill_rows(rows, n, cabi.ptr(x, cabi.f32p))
    assert not x[(rows - 1) * n:].any()          # the zero-norm row is present
    q = np.zeros(rows * (n // 128) * 98, np.uint8)
    y = np.zeros_like(x)
    for r in range(rows):
        oracle.tq6_quantize_row(cabi.ptr(x[r * n:], cabi.f32p), q[r * (n // 128) * 98:].ctypes.data, n)
    for r in range(rows):
        oracle.tq6_dequantize_row(q[r * (n // 128) * 98:].ctypes.data, cabi.ptr(y[r * n:], cabi.f32p), n)
    assert oracle.fnv1a(q.ctypes.data, q.nbytes, FNV0) == eenc
    assert oracle.fnv1a(y.ctypes.data, y.nbytes, FNV0) == edec
