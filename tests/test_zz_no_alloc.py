"""vcpp_paged_decode_noalloc (static split-K scratch, allocates nothing)
against vcpp_paged_decode with a workspace, through the C ABI: two calls in a
row, the second smaller, on every page dtype and both split modes.  The two
must agree bit for bit (same kernels, same split); the oracle bar applies too.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import DevPool, assert_close, dev

pytestmark = pytest.mark.gpu

TOL = {O.ORC_F32: (1e-4, 1e-4), O.ORC_F16: (2e-3, 1e-2), O.ORC_I8: (2e-3, 1e-2),
       O.ORC_FP8: (2e-3, 1e-2)}


def tables_for(seed, ctx, nb):
    nbs = [(c + 15) // 16 for c in ctx]
    perm = O.permutation(seed, nb)
    t = np.full((len(ctx), max(max(nbs), 1)), -1, np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    return t


def run_pair(dpool, pool, q, tables, ctx, partition, what, kind):
    qd, td, cd = dev(q), dev(tables), dev(ctx)
    mcl = int(ctx.max())
    ref = torch.full_like(qd, float("nan"))
    pyvcpp.paged_decode(dpool.pages, qd, ref, td, cd, mcl, 64, partition_size=partition)
    got = torch.full_like(qd, float("nan"))
    pyvcpp.paged_decode_noalloc(dpool.pages, qd, got, td, cd, mcl, 64, partition_size=partition)
    torch.cuda.synchronize()
    g, r = got.cpu().numpy(), ref.cpu().numpy()
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), "%s: noalloc differs from workspace" % what
    assert_close(g, O.decode(pool, q, tables, ctx, 64), *TOL[kind], what=what)


@pytest.mark.parametrize("partition", [0, 128])
@pytest.mark.parametrize("kind", [O.ORC_F32, O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_noalloc_matches_workspace_entry(cuda, kind, partition):
    nb = 2800
    pool = O.make_pool(kind, 900 + kind, nb, 8, 80)
    dpool = DevPool(pool)
    big = O.uniform_int(901, 24, 1, 2500).astype(np.int32)
    big[3] = 0
    small = np.array([700, 5, 16, 129], np.int32)
    for i, ctx in enumerate((big, small)):
        q = O.normal(910 + i, (len(ctx), 64, 80))
        run_pair(dpool, pool, q, tables_for(920 + i, ctx, nb), ctx, partition,
                 "noalloc kind=%d P=%d call %d" % (kind, partition, i), kind)


def test_noalloc_rejects_oversized_split(cuda):
    """A split whose partials exceed the static scratch is refused with a
    message, and nothing runs."""
    pool = O.make_pool(O.ORC_F16, 930, 8, 8, 80)
    dpool = DevPool(pool)
    n = 4096
    ctx = np.full(n, 16 * 1024, np.int32)
    need = pyvcpp.decode_workspace_size(dpool.pages, n, 64, int(ctx.max()), 64)
    assert need > (64 << 20)
    q = torch.zeros((n, 64, 80), dtype=torch.float32, device="cuda:0")
    with pytest.raises(pyvcpp.VcppError, match="static"):
        pyvcpp.paged_decode_noalloc(dpool.pages, q, q, dev(np.zeros((n, 1), np.int32)),
                                    dev(ctx), int(ctx.max()), 64, partition_size=64)
