"""Seeded synthetic inputs at the BASELINE.json distributions (shared by the GPU tests and bench.py).

Both sides of every parity check get the same fp16 / fp32 bits, so the generator only needs to be
deterministic for a given seed (numpy PCG64), not host-independent.

  C2/C3/C4 K rows: N(0,1) body, 2% of the channels (5 of 256) scaled x10, per-token norm lognormal(0, 0.3)
  V rows:          N(0,1)
  C1 K rows:       N(0,1), channels 3 and 77 scaled x12 (D = 128)
"""
import numpy as np


def kv_rows(n_pos, H, D, seed, outlier_frac=0.02, outlier_scale=10.0, tok_sigma=0.3):
    """K, V float32 [n_pos][H][D] drawn as above (before rotation)."""
    rng = np.random.default_rng(seed)
    K = rng.standard_normal((n_pos, H, D), dtype=np.float32)
    n_out = max(1, int(round(outlier_frac * D)))
    ch = rng.choice(D, size=n_out, replace=False)
    K[:, :, ch] *= np.float32(outlier_scale)
    K *= rng.lognormal(0.0, tok_sigma, size=(n_pos, H, 1)).astype(np.float32)
    V = rng.standard_normal((n_pos, H, D), dtype=np.float32)
    return K, V


def kv_rows_c1(seed=0, G=128, D=128):
    rng = np.random.default_rng(seed)
    K = rng.standard_normal((G, D), dtype=np.float32)
    K[:, 3] *= np.float32(12.0)
    K[:, 77] *= np.float32(12.0)
    V = rng.standard_normal((G, D), dtype=np.float32)
    return K, V


def round_trip_mse(x_bits, dec):
    """(MSE, MSE / mean square) of decoded rows against the fp16 rows sealed (configs[0]'s round-trip figure), in
    float64"""
    x = np.asarray(x_bits, np.uint16).view(np.float16).astype(np.float64).reshape(-1)
    d = np.asarray(dec, np.float32).astype(np.float64).reshape(-1)
    mse = float(np.mean((d - x) ** 2))
    return mse, mse / float(np.mean(x ** 2))


def f16_bits(x):
    """float32 array -> uint16 fp16 bits (numpy's conversion rounds to nearest even)."""
    return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


def fnv1a(buf, h=1469598103934665603):
    """FNV-1a 64 of a byte buffer (the reference's hashing protocol, tests/test_vectors.c:20-30)."""
    b = np.frombuffer(np.ascontiguousarray(buf).tobytes(), np.uint8)
    for x in b.tolist():
        h ^= x
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


# fp16 bit patterns that are not finite numbers: +-inf, +-quiet NaN, +-signalling NaN, NaNs with payloads
NONFINITE_HALVES = np.array([0x7C00, 0xFC00, 0x7E00, 0xFE00, 0x7C01, 0xFC01, 0x7E55, 0xFD23], np.uint16)


def nonfinite_groups(D, G=128, seed=0):
    """[(name, K, V)] of fp16 bit tiles [G][D] (token-major rows) holding infinities and NaNs of both signs:
    scattered specials, lone infinities (NaN only from inf - inf inside the seal), an all-inf row of each tile
    (K: one channel over every token; V: one token over every channel), a NaN first in a row, and tiles that are
    all +inf / all NaN."""
    rng = np.random.default_rng(seed)

    def body():
        return f16_bits(rng.standard_normal((G, D), dtype=np.float32))

    out = []
    K, V = body(), body()
    for X in (K, V):
        m = rng.random((G, D)) < 0.01
        X[m] = rng.choice(NONFINITE_HALVES, size=int(m.sum()))
    out.append(("scattered", K, V))
    K, V = body(), body()
    K[5, 7], K[90, 7], V[9, D - 56] = 0x7C00, 0xFC00, 0xFC00
    out.append(("lone_inf", K, V))
    K, V = body(), body()
    K[:, 3] = 0x7C00
    V[4, :] = 0xFC00
    out.append(("inf_row", K, V))
    K, V = body(), body()
    K[:, 11] = np.where(np.arange(G) % 2 == 0, 0x7C00, 0xFC00)
    V[17, :] = np.where(np.arange(D) % 3 == 0, 0xFC00, 0x7C00)
    out.append(("mixed_inf_row", K, V))
    K, V = body(), body()
    K[0, 10] = 0xFE00
    V[0, 0] = 0xFC01
    V[60, 0] = 0x7E55
    out.append(("nan_first", K, V))
    out.append(("all_inf", np.full((G, D), 0x7C00, np.uint16), np.full((G, D), 0xFC00, np.uint16)))
    out.append(("all_nan", np.full((G, D), 0xFE00, np.uint16), np.full((G, D), 0x7C01, np.uint16)))
    return out


def nonfinite_rows(n, D, seed=0):
    """float32 rows [n][D] for the tq6_0 / fp16 staging paths: N(0,1) rows with +-inf and NaNs of both signs
    in some 128-value blocks, blocks that are all inf, a NaN first in a block, and plain rows."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, D), dtype=np.float32)
    sp = np.array([np.inf, -np.inf, np.nan, -np.nan], np.float32)
    sp_bits = np.concatenate([sp.view(np.uint32), np.array([0x7F800001, 0xFF800001, 0x7FC00055], np.uint32)])
    for r in range(n):
        kind = r % 6
        if kind == 0:
            x[r, rng.integers(0, D)] = np.inf
        elif kind == 1:
            x[r, rng.integers(0, D)] = -np.inf
        elif kind == 2:
            x[r].view(np.uint32)[rng.integers(0, D, 3)] = rng.choice(sp_bits, 3)
        elif kind == 3:
            x[r, :128] = np.inf
        elif kind == 4:
            x[r].view(np.uint32)[0] = 0xFFC00000
    return x


def f16_isnan(h):
    h = np.asarray(h, np.uint16)
    return ((h & 0x7C00) == 0x7C00) & ((h & 0x03FF) != 0)


def halves_equal_nan_unsigned(a, b):
    """fp16 bit arrays equal, where a NaN equals any NaN: IEEE 754 (section 6.3) leaves the sign of a NaN result
    unspecified, and which operand's NaN an x86 add or multiply returns depends on how the compiler ordered the
    operands (two builds of the reference differ there)."""
    a, b = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
    return (a == b) | (f16_isnan(a) & f16_isnan(b))


def floats_equal_nan_unsigned(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def record_mismatch(lay, a, b):
    """byte offsets where two records differ: payload bytes exactly, the fp16 scale arrays up to NaN signs"""
    a, b = np.asarray(a, np.uint8), np.asarray(b, np.uint8)
    p = lay.k_scale
    bad = list(np.nonzero(a[:p] != b[:p])[0])
    ok = halves_equal_nan_unsigned(a[p:].view(np.uint16), b[p:].view(np.uint16))
    bad += list(p + 2 * np.nonzero(~ok)[0])
    return np.array(bad, np.int64)


def tq6_mismatch(a, b):
    """byte offsets where two arrays of 98-byte tq6_0 blocks differ: codes exactly, the fp16 norm up to NaN signs"""
    a, b = np.asarray(a, np.uint8).reshape(-1, 98), np.asarray(b, np.uint8).reshape(-1, 98)
    bad = np.nonzero((a[:, 2:] != b[:, 2:]).any(axis=1) |
                     ~halves_equal_nan_unsigned(a[:, :2].copy().view(np.uint16)[:, 0],
                                                b[:, :2].copy().view(np.uint16)[:, 0]))[0]
    return bad * 98
