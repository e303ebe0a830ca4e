"""The physics FLOP table of g1.cu_amd/roofline.py against the operation-counting instantiation of
the oracle (oracle/flop_count.cpp): per contact count c = 0..8 at 8 PGS sweeps, the smallest count
over sampled contact states equals the table; the table's PGS-sweep term equals the counted
difference of two sweep counts (and its closed form 2n^2 + 3n, n = 4c rows); the counted run
reproduces the fp32 oracle's contact counts (the same algorithm runs)."""
import numpy as np

import roofline


def _states(orc, n=900, seed=2):
    import configs
    import g1_model as gm
    qp, qv, _ = configs.config2(lambda q: orc.fk(q, dtype=np.float64), n=n, seed=seed)
    rng = np.random.default_rng(1)
    tg = np.clip(gm.qpos_stand[7:][None] + 0.1 * rng.uniform(-1, 1, (n, 29)), gm.act_ctrl_lo, gm.act_ctrl_hi)
    return qp.astype(np.float32), qv.astype(np.float32), tg.astype(np.float32)


def test_flop_table_matches_counting_oracle(orc):
    qp, qv, tg = _states(orc)
    _, _, _, nref = orc.substep(qp, qv, tg, pgs=8, mu=0.6)
    per_c = {}
    for i in range(len(qp)):
        nc, cnt = orc.count_substep(qp[i], qv[i], tg[i], pgs=8)
        assert nc == nref[i]
        per_c.setdefault(nc, []).append(orc.flops_of(cnt))
    assert sorted(per_c) == list(range(9))
    for c in range(9):
        v = np.array(per_c[c])
        assert int(v.min()) == roofline.FLOPS_P8[c], (c, int(v.min()))
        assert v.max() - v.min() <= 5e-4 * v.min()
    assert orc.flops_of(orc.count_step_overhead()) == roofline.STEP_OVERHEAD_FLOPS


def test_pgs_sweep_term(orc):
    qp, qv, tg = _states(orc, n=120, seed=3)
    seen = set()
    for i in range(len(qp)):
        _, c8 = orc.count_substep(qp[i], qv[i], tg[i], pgs=8)
        nc, c3 = orc.count_substep(qp[i], qv[i], tg[i], pgs=3)
        n = 4 * nc
        assert orc.flops_of(c8) - orc.flops_of(c3) == 5 * (2 * n * n + 3 * n)
        assert roofline.flops_per_world_substep(nc, 3) == roofline.FLOPS_P8[nc] - 5 * (2 * n * n + 3 * n)
        seen.add(nc)
    assert len(seen) >= 5
