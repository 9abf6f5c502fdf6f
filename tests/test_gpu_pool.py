"""Per-sequence cache stress on the paged pool (the configs[4] workload, scaled down): sequences of
random-length prompts share one record pool; decode rounds at width 4 commit through the adaptive-tail
policy; one sequence is truncated into its sealed body, another saved to a state stream and restored.
Sampled records are re-sealed on the CPU and must be byte-identical; sampled attention rows must agree
with the oracle's loop within max-abs 1e-3 + rel 1e-3."""
import sys

import pytest

import cabi
import inputs
import pool_check

sys.path.insert(0, cabi.PKG)
import pool_stress  # noqa: E402
import sjk  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return sjk.load()


@pytest.fixture(scope="module")
def dev():
    d = sjk.Device()
    yield d
    d.free_all()


@pytest.mark.parametrize("bk,bv,body,batched", [(3, 3, 1, True), (4, 4, 0, True), (3, 3, 1, False)],
                         ids=["3/3t-batched", "4/4s-batched", "3/3t-per-call"])
def test_pool_stress_small(oracle, lib, dev, bk, bv, body, batched):
    ps, rep = pool_stress.run(lib, dev, inputs.kv_rows, n_layers=2, n_seq=3, bk=bk, bv=bv, body=body, batched=batched,
                              prompt=(700, 1500), steps=200, width=4, tail=256, tail_max=512, trunc_back=700,
                              log=lambda *a: print(*a, flush=True))
    try:
        print(rep, flush=True)
        assert rep["commits"] >= ps.n_seq
        tr = rep["truncate"]
        assert tr["kept"] <= tr["to"] and tr["B_after"] <= tr["kept"]
        assert tr["B_after"] < tr["B_before"]                       # the cut reached into the sealed body
        sr = rep["save_restore"]
        assert sr["stream_equal"] and sr["attention_equal"] and sr["async_save"]["stream_equal_sync"]
        assert rep["rounds"] >= 200                 # (the restore runs one round more when the save took the rest)
        for s in range(ps.n_seq):
            seq = ps.seqs[s]
            assert seq.n == rep["final_positions"][s]
            n_groups = (seq.pol.B - ps.S) // ps.G
            assert n_groups > 0
            # first and last sealed group of every sequence and layer (for the truncated sequence the last
            # one was sealed from rows stored after the cut)
            for il in range(ps.n_layers):
                groups = sorted({0, n_groups - 1})
                eq = pool_check.check_records(oracle, ps, s, il, groups)
                assert eq == len(groups) * ps.H, (s, il, groups, eq)
                rows = [(iq, hq) for iq in range(ps.width) for hq in range(0, ps.n_head, 3)]
                worst = pool_check.check_attention(oracle, ps, s, il, rows)
                assert worst <= 1.0, (s, il, worst)
    finally:
        ps.free()
