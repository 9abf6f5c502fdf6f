"""Adaptive-tail journal policy of the oracle (sj_kvarn.h:1315-1407).

Fuzzed against an independent Python statement of the per-ubatch rule, with the invariants an engine relies
on (whole groups, tail kept exact, ring never overrun), random idle steps and truncations, in the manner of
the reference's tests/test_policy.c:31-99; plus its deterministic default-schedule and idle tables
(tests/test_policy.c:101-135).
"""
import ctypes as C

import pytest

import cabi

NO_POS = 0xFFFFFFFF


class PyPolicy:
    """Independent statement of the commit rule: a commit is due when the unsealed span reaches tail_max
    (or always for a fixed tail, or while draining); it seals to the group boundary at or below
    pos0 - tail; decode-sized ubatches seal at most flush_chunk groups."""

    def __init__(self, sink, tail, tail_max, G, chunk):
        self.sink, self.tail, self.tail_max, self.G, self.chunk = sink, tail, tail_max, G, chunk
        self.B = self.pending = sink
        self.draining = 0

    def begin(self, pos0, n):
        due = self.tail_max == 0 or self.draining or (pos0 > self.B and pos0 - self.B >= self.tail_max)
        self.pending = self.B
        self.draining = 0
        if due and pos0 > self.sink + self.tail:
            target = max(self.B, self.sink + self.G * ((pos0 - self.tail - self.sink) // self.G))
            if self.tail_max > 0 and self.chunk > 0 and n < self.G and target > self.B + self.G * self.chunk:
                target = self.B + self.G * self.chunk
                self.draining = 1
            self.pending = target
        return self.pending


class Rng:
    def __init__(self, s):
        self.s = s

    def __call__(self):
        s = self.s
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        self.s = s
        return (s >> 11) & 0xFFFFFFFF


@pytest.mark.parametrize("tail,tail_max", [(4096, 8192), (4096, 0), (256, 512), (128, 128), (0, 0), (512, 1024)])
@pytest.mark.parametrize("chunk", [0, 1, 2])
def test_policy_fuzz(oracle, tail, tail_max, chunk):
    rnd = Rng(88172645463325252 + tail * 7 + tail_max + chunk)
    G, sink = 128, 128
    for trial in range(6):
        nub = 1 + rnd() % 512
        cap = oracle.ring_capacity(tail, tail_max, G, nub)
        assert cap % 128 == 0 and cap >= max(tail, tail_max) + G + 2 * nub
        p = cabi.Policy()
        oracle.policy_init(C.byref(p), sink, tail, tail_max, G, chunk)
        ref = PyPolicy(sink, tail, tail_max, G, chunk)
        pos = 0
        while pos < 20000:
            n = 1 + rnd() % 8 if rnd() % 4 else 1 + rnd() % nub
            B_prev = p.B
            pend = oracle.policy_begin_ubatch(C.byref(p), pos, n)
            assert pend == ref.begin(pos, n) and p.draining == ref.draining
            if pend > B_prev:
                assert (pend - sink) % G == 0
                assert pos - pend >= tail
            oracle.policy_commit(C.byref(p))
            ref.B = ref.pending
            assert pos + n <= B_prev + cap, "unsealed rows would overrun the ring"
            pos += n
            if tail_max > 0 and rnd() % 64 == 0:
                keep = 0 if rnd() % 2 else rnd() % 12000
                margin = max(keep, tail)
                t = oracle.policy_idle(C.byref(p), pos, keep)
                if t > p.B:
                    assert pos - t >= margin and (t - sink) % G == 0
                    oracle.policy_commit(C.byref(p))
                ref.B = ref.pending = p.B
                ref.draining = p.draining
            if rnd() % 389 == 0:
                back = rnd() % (min(pos, 1500) + 1)
                cut, B_before = pos - back, p.B
                dropped = C.c_uint32(0)
                floor_q = oracle.policy_trunc_floor(C.byref(p), cut)
                res = oracle.policy_truncate(C.byref(p), cut, C.byref(dropped))
                assert res != NO_POS and res == floor_q and res <= cut and cut - res <= G - 1
                if cut >= B_before or cut <= sink:
                    assert res == cut
                else:
                    assert (res - sink) % G == 0
                if cut >= B_before:
                    assert p.B == B_before and dropped.value == 0
                else:
                    nb = max(res, sink)
                    assert p.B == nb == p.B_pending == p.B_prev and not p.draining
                    assert dropped.value == (B_before - nb) // G
                ref.B = ref.pending = p.B
                ref.draining = p.draining
                pos = res


def test_default_decode_schedule(oracle):
    """One token at a time with the defaults: 23 commits per 100K tokens, longest tail 8191
    (tests/test_policy.c:101-112 and its printed result)."""
    p = cabi.Policy()
    oracle.policy_init(C.byref(p), 128, 4096, 8192, 128, 0)
    commits = maxspan = 0
    for pos in range(100000):
        if oracle.policy_begin_ubatch(C.byref(p), pos, 1) > p.B:
            commits += 1
        oracle.policy_commit(C.byref(p))
        if pos > p.B:
            maxspan = max(maxspan, pos - p.B)
    assert commits == 23 and maxspan == 8191
    # the C4 attention shape: N = 100000 reached this way leaves B = 94336
    assert p.B == 94336


@pytest.mark.parametrize("B,end,keep,want", [(128, 1000, 0, 640), (128, 1000, 100, 640), (128, 1000, 256, 640),
                                             (128, 1000, 400, 512), (128, 1000, 872, 128), (640, 1000, 400, 640)])
def test_idle_margin(oracle, B, end, keep, want):
    p = cabi.Policy()
    oracle.policy_init(C.byref(p), 128, 256, 512, 128, 0)
    p.B = p.B_prev = p.B_pending = B
    got = oracle.policy_idle(C.byref(p), end, keep)
    assert got == want


def test_truncate_refused_while_pending(oracle):
    p = cabi.Policy()
    oracle.policy_init(C.byref(p), 128, 256, 512, 128, 0)
    assert oracle.policy_begin_ubatch(C.byref(p), 1000, 1) > p.B
    assert oracle.policy_truncate(C.byref(p), 500, None) == NO_POS
