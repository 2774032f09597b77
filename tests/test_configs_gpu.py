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


@pytest.fixture(scope="module")
def config5():
    """128 decode sequences (ctx U[1024, 8192]) plus 4 prefill chunks of 512
    tokens on 1024-token prefixes, int8 pages with fp16 scales; oracle outputs
    of every decode and of sampled prefill rows."""
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
    ref = fp32_view(pool)
    want_d = O.decode(ref, qd, dtab, dctx, 64, nthreads=NTHREADS)
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([rng.integers(0, 2048, 96), q_start[:-1], q_start[1:] - 1]))
    want_p = oracle_prefill_rows(ref, qp.astype(np.float32), ptab, q_start, prefix, 64, rows,
                                 nthreads=NTHREADS)
    return dict(pool=pool, dctx=dctx, dtab=dtab, ptab=ptab, qd=qd, q_start=q_start, prefix=prefix,
                qp=qp, want_d=want_d, rows=rows, want_p=want_p)


@pytest.mark.parametrize("mode", ["two_launches", "mixed_step", "mixed_step_fused"])
def test_config5_int8_mixed_step(cuda, config5, mode, monkeypatch):
    """BASELINE config 5 as one step: decode then prefill on one stream, or
    vcpp_paged_mixed_step (two launches, or with VCPP_MIXED_FUSED=1 one fused
    launch + the decode merge)."""
    monkeypatch.setenv("VCPP_MIXED_FUSED", "1" if mode == "mixed_step_fused" else "0")
    c = config5
    dp = DevPool(c["pool"])
    qdd = dev(c["qd"])
    out_d = torch.full_like(qdd, float("nan"))
    out_p = torch.full(c["qp"].shape, float("nan"), dtype=torch.float32, device="cuda:0")
    args_p = (dev(c["qp"].view(np.uint16)), out_p, dev(c["ptab"]), dev(c["q_start"]), dev(c["prefix"]), 512)
    if mode == "two_launches":
        pyvcpp.paged_decode(dp.pages, qdd, out_d, dev(c["dtab"]), dev(c["dctx"]), int(c["dctx"].max()), 64)
        pyvcpp.paged_prefill(dp.pages, *args_p, 64)
    else:
        pyvcpp.paged_mixed_step(dp.pages, qdd, out_d, dev(c["dtab"]), dev(c["dctx"]), int(c["dctx"].max()),
                                *args_p, 64)
    torch.cuda.synchronize()
    assert_close(out_d.cpu().numpy(), c["want_d"], *TOL, what="config5 decode (%s)" % mode)
    assert_close(out_p.cpu().numpy()[c["rows"]], c["want_p"], *TOL, what="config5 prefill rows (%s)" % mode)
