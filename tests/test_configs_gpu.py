"""BASELINE configs 4 and 5 at full size on the GPU, checked against the
oracle (fp16 / int8 pages: atol 2e-3, rtol 1e-2).

The oracle reads an fp32 pool holding exactly the values the fp16 / int8
pages encode (oracle_lib.Pool.dequant): the same arithmetic as reading the
encoded pages, without decoding every element on every pass."""
import os

import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import DevPool, assert_close, dev, gpu_decode, oracle_prefill_rows

pytestmark = pytest.mark.gpu
TOL = (2e-3, 1e-2)
NTHREADS = min(16, os.cpu_count() or 1)


def scattered_tables(seed, ctx, num_blocks):
    nbs = [(int(c) + 15) // 16 for c in ctx]
    perm = O.permutation(seed, num_blocks)
    t = np.full((len(ctx), max(nbs)), -1, np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    return t


def fp32_view(pool):
    k, v = pool.dequant()
    return O.Pool(O.ORC_F32, k, v)


@pytest.fixture(scope="module")
def config4():
    """16 sequences x 32768 tokens, fp16 pages scattered over a pool of 1.25x
    the tokens, q/K/V ~ N(0,1)."""
    ctx = np.full(16, 32768, np.int32)
    nb = int(1.25 * ctx.sum() / 16)
    pool = O.make_pool(O.ORC_F16, 401, nb, 8, 80)
    q = O.normal(402, (16, 64, 80))
    tables = scattered_tables(403, ctx, nb)
    want = O.decode(fp32_view(pool), q, tables, ctx, 64, nthreads=NTHREADS)
    return pool, q, tables, ctx, want


@pytest.mark.parametrize("partition", [256, 0])
def test_config4_long_context(cuda, config4, partition):
    """Split-K over 256-token partitions (the config's statement) and the
    balanced split; both merged by the log-sum-exp kernel."""
    pool, q, tables, ctx, want = config4
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64, partition_size=partition)
    assert_close(got, want, *TOL, what="config4 P=%d" % partition)


def test_config5_int8_mixed_step(cuda):
    """128 decode sequences (ctx U[1024, 8192]) plus 4 prefill chunks of 512
    tokens on 1024-token prefixes, int8 pages with fp16 scales, run as one
    step (decode launch, then prefill launch, same stream)."""
    dctx = O.uniform_int(501, 128, 1024, 8192)
    plen = np.full(4, 1024 + 512, np.int32)
    nb = int(np.ceil(1.25 * (dctx.sum() + plen.sum()) / 16))
    pool = O.make_pool(O.ORC_I8, 502, nb, 8, 80)
    alltab = scattered_tables(503, np.concatenate([dctx, plen]), nb)
    dtab, ptab = alltab[:128], alltab[128:]
    qd = O.normal(504, (128, 64, 80))
    q_start = np.arange(0, 4 * 512 + 1, 512, dtype=np.int32)
    prefix = np.full(4, 1024, np.int32)
    qp = O.normal(505, (4 * 512, 64, 80)).astype(np.float16)

    dp = DevPool(pool)
    qdd = dev(qd)
    out_d = torch.full_like(qdd, float("nan"))
    out_p = torch.full(qp.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    pyvcpp.paged_decode(dp.pages, qdd, out_d, dev(dtab), dev(dctx), int(dctx.max()), 64)
    pyvcpp.paged_prefill(dp.pages, dev(qp.view(np.uint16)), out_p, dev(ptab), dev(q_start),
                         dev(prefix), 512, 64)
    torch.cuda.synchronize()

    ref = fp32_view(pool)
    want_d = O.decode(ref, qd, dtab, dctx, 64, nthreads=NTHREADS)
    assert_close(out_d.cpu().numpy(), want_d, *TOL, what="config5 decode")
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([rng.integers(0, 2048, 96), q_start[:-1], q_start[1:] - 1]))
    want_p = oracle_prefill_rows(ref, qp.astype(np.float32), ptab, q_start, prefix, 64, rows,
                                 nthreads=NTHREADS)
    assert_close(out_p.cpu().numpy()[rows], want_p, *TOL, what="config5 prefill rows")
