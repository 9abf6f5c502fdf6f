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
