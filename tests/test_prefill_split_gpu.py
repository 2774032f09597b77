"""GPU parity of the key-split chunked prefill (vcpp_paged_prefill_split)
against the CPU oracle's per-position semantics, on the shapes it exists for
(few chunks on long prefixes, where the keys of each query tile are cut over
several workgroups and merged by log-sum-exp).

Tolerance: max-abs error <= 2e-3 and normwise relative error <= 1e-2, as for
the unsplit prefill (int8 on std-2 data: 4e-3).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import DevPool, assert_close, dev, gpu_prefill, gpu_prefill_split
from test_prefill_gpu import make_case
import pyvcpp

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
@pytest.mark.parametrize("D", [64, 80, 128])
def test_split_long_prefix(cuda, kind, D):
    """One chunk on a long prefix: an odd block count, a chunk that is not a
    multiple of the query tile, std-2 scores (many running-max moves in every
    part), and early query tiles whose leading parts hold no keys."""
    prefix, chunk = [6001], [97]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 700 + D + kind, prefix, chunk, 16, 2, D,
                                                     std=2.0)
    want = O.prefill(pool, q32, tables, q_start, pre, 16)
    got, split = gpu_prefill_split(DevPool(pool), q16, tables, q_start, pre, 16)
    assert split, "shape was meant to split"
    atol = ATOL * 2.0 if kind == O.ORC_I8 else ATOL
    assert_close(got, want, atol, RTOL, what="split D=%d kind=%d" % (D, kind))


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_FP8])
def test_split_mixed_chunks(cuda, kind):
    """Chunks of different prefixes and lengths in one call, including an
    empty chunk, a prefix of zero, and a chunk whose tiles span fewer key
    blocks than there are parts."""
    prefix, chunk = [4000, 0, 33, 2500], [40, 300, 0, 1]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 720 + kind, prefix, chunk, 64, 8)
    want = O.prefill(pool, q32, tables, q_start, pre, 64)
    got, split = gpu_prefill_split(DevPool(pool), q16, tables, q_start, pre, 64)
    assert split
    assert_close(got, want, ATOL, RTOL, what="split mixed kind=%d" % kind)


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8])
def test_split_skips_invalid_blocks(cuda, kind):
    prefix, chunk = [3000, 1500], [20, 64]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 730 + kind, prefix, chunk, 8, 1)
    tables[0, 5] = -1          # a prefix page missing, inside an early part
    tables[1, 90] = 10 ** 6    # an id past the pool, near a part boundary
    want = O.prefill(pool, q32, tables, q_start, pre, 8)
    got, split = gpu_prefill_split(DevPool(pool), q16, tables, q_start, pre, 8)
    assert split
    assert_close(got, want, ATOL, RTOL, what="split invalid blocks kind=%d" % kind)


def test_split_matches_unsplit_and_reuses_workspace(cuda):
    """Split and unsplit prefill agree; a second call on a smaller shape with
    the first call's workspace (stale contents) gives the oracle's answer."""
    prefix, chunk = [5000, 4100], [64, 128]
    pool, q16, q32, tables, q_start, pre = make_case(O.ORC_F16, 740, prefix, chunk, 32, 4)
    dp = DevPool(pool)
    need = pyvcpp.prefill_workspace_size(dp.pages, 2, 128, 5000, 32)
    assert need > 0
    ws = torch.full((need,), 0x7f, dtype=torch.uint8, device="cuda:0")
    got, _ = gpu_prefill_split(dp, q16, tables, q_start, pre, 32, workspace=ws)
    ref = gpu_prefill(dp, q16, tables, q_start, pre, 32)
    assert_close(got, ref, ATOL, RTOL, what="split vs unsplit")
    want = O.prefill(pool, q32, tables, q_start, pre, 32)
    assert_close(got, want, ATOL, RTOL, what="split vs oracle")
    # Smaller second call on the same workspace.
    p2, c2 = [2100], [50]
    pool2, q16b, q32b, tb2, qs2, pre2 = make_case(O.ORC_F16, 741, p2, c2, 32, 4)
    got2, split2 = gpu_prefill_split(DevPool(pool2), q16b, tb2, qs2, pre2, 32, workspace=ws)
    assert split2
    assert_close(got2, O.prefill(pool2, q32b, tb2, qs2, pre2, 32), ATOL, RTOL, what="second call")


def test_split_short_prefix_needs_no_workspace(cuda):
    prefix, chunk = [10, 0], [30, 200]
    pool, q16, q32, tables, q_start, pre = make_case(O.ORC_F16, 750, prefix, chunk, 64, 8)
    got, split = gpu_prefill_split(DevPool(pool), q16, tables, q_start, pre, 64)
    assert not split
    assert_close(got, O.prefill(pool, q32, tables, q_start, pre, 64), ATOL, RTOL, what="unsplit")


def test_split_rejects_small_workspace(cuda):
    prefix, chunk = [6000], [16]
    pool, q16, q32, tables, q_start, pre = make_case(O.ORC_F16, 760, prefix, chunk, 8, 1)
    dp = DevPool(pool)
    need = pyvcpp.prefill_workspace_size(dp.pages, 1, 16, 6000, 8)
    assert need > 0
    ws = torch.empty(need - 1, dtype=torch.uint8, device="cuda:0")
    out = torch.empty(q16.shape, dtype=torch.float32, device="cuda:0")
    with pytest.raises(RuntimeError):
        pyvcpp.paged_prefill_split(dp.pages, dev(q16), out, dev(tables), dev(q_start), dev(pre), 16, 6000, 8,
                                   workspace=ws)


@pytest.mark.parametrize("split", [False, True])
def test_chunk_longer_than_max_chunk_len(cuda, split):
    """A caller error: chunk 0 holds 200 rows but max_chunk_len says 64.
    Rows the grid does not reach keep their previous contents (NaN here),
    every other row equals the oracle; the split path's merge does not write
    stale workspace rows into the uncovered ones (its workspace holds rows
    below num_chunks * max_chunk_len only, so there the rest stay unwritten
    too)."""
    prefix, chunk = [4000, 3000], [200, 40]
    pool, q16, q32, tables, q_start, pre = make_case(O.ORC_F16, 760, prefix, chunk, 16, 2)
    dp = DevPool(pool)
    out = torch.full(q16.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    args = (dp.pages, dev(q16), out, dev(np.asarray(tables, np.int32)), dev(np.asarray(q_start, np.int32)),
            dev(np.asarray(pre, np.int32)), 64)
    if split:
        need = pyvcpp.prefill_workspace_size(dp.pages, 2, 64, 4000, 16)
        assert need > 0
        ws = torch.full((need,), 0x3f, dtype=torch.uint8, device="cuda:0")  # stale finite values
        pyvcpp.paged_prefill_split(*args, 4000, 16, workspace=ws)
    else:
        pyvcpp.paged_prefill(*args, 16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = O.prefill(pool, q32, tables, q_start, pre, 16)
    rows_nan = np.isnan(got).all(axis=(1, 2))
    assert (np.isnan(got).any(axis=(1, 2)) == rows_nan).all(), "a row is partly written"
    assert rows_nan[:128].all(), "rows before the chunk's reachable tiles were written"
    if not split:  # (the split path stores only rows below num_chunks * max_chunk_len = 128)
        assert not rows_nan[192:200].any(), "the chunk's last tile was not computed"
    assert_close(got[~rows_nan], want[~rows_nan], ATOL, RTOL, what="written rows, split=%s" % split)
