"""vcpp_paged_mixed_step: a scheduler step carrying decodes and prefill chunks
(src/scheduler.h:14-23, served together at src/paged_engine.cpp:254-269),
checked against the oracle's decode (src/paged_attention.cpp:11-90) and
per-position prefill (src/paged_engine.cpp:348-384) on the same pages: both
the default two launches and the opt-in fused single launch
(VCPP_MIXED_FUSED=1, where the shape allows it)."""
import os

import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import DevPool, assert_close, dev, prefill_tables

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-2


def mixed_case(kind, seed, dctx, prefix, chunk, H, Hkv, D=80):
    plen = [p + n for p, n in zip(prefix, chunk)]
    lens = list(dctx) + plen
    nb = sum((l + 15) // 16 for l in lens) + 8
    pool = O.make_pool(kind, seed, nb, Hkv, D)
    tables = prefill_tables(seed + 1, [max(l, 1) for l in lens], nb)
    dtab, ptab = tables[:len(dctx)], tables[len(dctx):]
    qd = O.normal(seed + 2, (len(dctx), H, D))
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    qp = O.normal(seed + 3, (int(q_start[-1]), H, D)).astype(np.float16)
    return pool, np.asarray(dctx, np.int32), dtab, qd, ptab, q_start, np.asarray(prefix, np.int32), qp


def run_mixed(pool, dctx, dtab, qd, ptab, q_start, prefix, qp, H, fused=True):
    dp = DevPool(pool)
    qdd = dev(qd)
    out_d = torch.full_like(qdd, float("nan"))
    out_p = torch.full(qp.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    old = os.environ.get("VCPP_MIXED_FUSED")
    os.environ["VCPP_MIXED_FUSED"] = "1" if fused else "0"
    try:
        pyvcpp.paged_mixed_step(dp.pages, qdd, out_d, dev(dtab), dev(dctx), int(dctx.max()),
                                dev(qp.view(np.uint16)), out_p, dev(ptab), dev(q_start), dev(prefix),
                                int(np.diff(q_start).max()), H)
        torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ["VCPP_MIXED_FUSED"]
        else:
            os.environ["VCPP_MIXED_FUSED"] = old
    return out_d.cpu().numpy(), out_p.cpu().numpy()


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
@pytest.mark.parametrize("heads", [(64, 8), (32, 4), (8, 1)])
def test_mixed_small(cuda, kind, heads, fused):
    """Ragged decodes (empty, one token, a partial tile, long) beside ragged
    prefill chunks; (8, 1) heads have no fused step and take two launches."""
    H, Hkv = heads
    dctx = [0, 1, 17, 300, 1000, 33, 2047]
    prefix, chunk = [0, 19, 200, 64], [1, 70, 37, 129]
    pool, dctx, dtab, qd, ptab, q_start, pre, qp = mixed_case(kind, 700 + H + kind, dctx, prefix, chunk, H, Hkv)
    got_d, got_p = run_mixed(pool, dctx, dtab, qd, ptab, q_start, pre, qp, H, fused)
    assert_close(got_d, O.decode(pool, qd, dtab, dctx, H), ATOL, RTOL,
                 what="mixed decode H=%d Hkv=%d kind=%d fused=%d" % (H, Hkv, kind, fused))
    assert_close(got_p, O.prefill(pool, qp.astype(np.float32), ptab, q_start, pre, H), ATOL, RTOL,
                 what="mixed prefill H=%d Hkv=%d kind=%d fused=%d" % (H, Hkv, kind, fused))


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8])
def test_mixed_skip_rules(cuda, kind):
    """Invalid and out-of-pool block ids are skipped on both sides."""
    dctx = [64, 200, 5]
    prefix, chunk = [48, 0], [40, 70]
    pool, dctx, dtab, qd, ptab, q_start, pre, qp = mixed_case(kind, 740, dctx, prefix, chunk, 64, 8)
    dtab[1, 3] = -1
    dtab[0, 0] = 10 ** 6
    ptab[0, 1] = -1
    ptab[1, 2] = 10 ** 6
    got_d, got_p = run_mixed(pool, dctx, dtab, qd, ptab, q_start, pre, qp, 64)
    assert_close(got_d, O.decode(pool, qd, dtab, dctx, 64), ATOL, RTOL, what="mixed skip decode")
    assert_close(got_p, O.prefill(pool, qp.astype(np.float32), ptab, q_start, pre, 64), ATOL, RTOL,
                 what="mixed skip prefill")


def test_mixed_one_side_empty(cuda):
    """No prefill chunks, or no decodes: the step is the other call alone."""
    dctx = [100, 3000]
    prefix, chunk = [10], [50]
    pool, dctx, dtab, qd, ptab, q_start, pre, qp = mixed_case(O.ORC_F16, 760, dctx, prefix, chunk, 64, 8)
    dp = DevPool(pool)
    qdd = dev(qd)
    out_d = torch.full_like(qdd, float("nan"))
    pyvcpp.paged_mixed_step(dp.pages, qdd, out_d, dev(dtab), dev(dctx), int(dctx.max()), None, None, None,
                            None, None, 0, 64)
    out_p = torch.full(qp.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    pyvcpp.paged_mixed_step(dp.pages, None, None, None, None, 0, dev(qp.view(np.uint16)), out_p, dev(ptab),
                            dev(q_start), dev(pre), int(np.diff(q_start).max()), 64)
    torch.cuda.synchronize()
    assert_close(out_d.cpu().numpy(), O.decode(pool, qd, dtab, dctx, 64), ATOL, RTOL, what="mixed decode only")
    assert_close(out_p.cpu().numpy(), O.prefill(pool, qp.astype(np.float32), ptab, q_start, pre, 64),
                 ATOL, RTOL, what="mixed prefill only")


@pytest.mark.parametrize("case", range(6))
def test_mixed_random(cuda, case):
    """Seeded random steps through the default path (decode, then the prefill
    beside the decode's merge on the side stream): page dtype, heads, head
    dim, ragged decode contexts and prefill chunks drawn together."""
    rng = np.random.default_rng(9100 + case)
    kind = int(rng.choice([O.ORC_F16, O.ORC_I8, O.ORC_FP8]))
    H, Hkv = [(64, 8), (32, 4), (16, 2), (24, 8)][int(rng.integers(4))]
    D = int(rng.choice([64, 80, 128]))
    nd = int(rng.integers(1, 40))
    dctx = rng.integers(0, 3000, nd)
    dctx[rng.random(nd) < 0.1] = 0
    nc = int(rng.integers(1, 5))
    prefix = rng.integers(0, 1500, nc)
    chunk = rng.integers(1, 200, nc)
    print("mixed case %d: kind %d H %d Hkv %d D %d decodes %d (tokens %d) chunks %s prefixes %s"
          % (case, kind, H, Hkv, D, nd, int(dctx.sum()), list(chunk), list(prefix)), flush=True)
    pool, dctx, dtab, qd, ptab, q_start, pre, qp = mixed_case(kind, 9200 + case, list(dctx), list(prefix),
                                                              list(chunk), H, Hkv, D)
    got_d, got_p = run_mixed(pool, dctx, dtab, qd, ptab, q_start, pre, qp, H, fused=False)
    assert_close(got_d, O.decode(pool, qd, dtab, dctx, H), ATOL, RTOL, what="mixed random %d decode" % case)
    assert_close(got_p, O.prefill(pool, qp.astype(np.float32), ptab, q_start, pre, H), ATOL, RTOL,
                 what="mixed random %d prefill" % case)
