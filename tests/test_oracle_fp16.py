"""fp16 conversion of the oracle (sj_kvarn.h:693-731).

Pinned three ways: every half round-trips (tests/test_fp16.c:28-33 of the reference); every finite float
in and around the half range converts like numpy's IEEE round-to-nearest-even float16 cast (an
independent library routine); and every
one of the 2^32 float bit patterns converts exactly like the compiled reference (where oracle/_ref is built).
"""
import ctypes as C
from concurrent.futures import ThreadPoolExecutor

import numpy as np

import cabi

CHUNK = 1 << 24


def _conv(api, bits):
    x = bits.view(np.float32)
    out = np.zeros(x.size * 2, np.uint8)
    api.stage_row(1, cabi.ptr(x, cabi.f32p), out.ctypes.data, x.size)   # F16 staging = f32_to_f16 per value
    return out.view(np.uint16)


def test_every_half_round_trips(oracle):
    h = np.arange(65536, dtype=np.uint16)
    f = np.zeros(65536, np.float32)
    oracle.unstage_row(1, h.ctypes.data, cabi.ptr(f, cabi.f32p), 65536)
    back = _conv(oracle, f.view(np.uint32))
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    assert np.array_equal(back[~nan], h[~nan])
    assert np.array_equal(f[~nan], h[~nan].view(np.float16).astype(np.float32))
    assert np.all(back[nan] == ((h[nan] & 0x8000) | 0x7E00))


def test_all_floats_match_numpy_rne(oracle):
    def run(i):
        bits = np.arange(i * CHUNK, (i + 1) * CHUNK, dtype=np.uint64).astype(np.uint32)
        got = _conv(oracle, bits)
        x = bits.view(np.float32)
        with np.errstate(over="ignore", invalid="ignore"):
            want = x.astype(np.float16).view(np.uint16)
        nan = np.isnan(x)
        want = np.where(nan, ((bits >> 16) & 0x8000) | 0x7E00, want).astype(np.uint16)
        return int(np.count_nonzero(got != want))
    # the whole half range (float exponents 0x66..0x8F) plus every 16th chunk elsewhere
    chunks = sorted(set(range(0x33, 0x48)) | set(range(0, 256, 16)))
    with ThreadPoolExecutor(8) as ex:
        bad = sum(ex.map(run, chunks))
    assert bad == 0


def test_all_floats_match_reference(oracle, ref):
    def run(i):
        bits = np.arange(i * CHUNK, (i + 1) * CHUNK, dtype=np.uint64).astype(np.uint32)
        return int(np.count_nonzero(_conv(oracle, bits) != _conv(ref, bits)))
    with ThreadPoolExecutor(8) as ex:
        bad = sum(ex.map(run, range(256)))
    assert bad == 0
