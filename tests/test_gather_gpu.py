"""Block-table gather indices, element by element.

The checker build of the library (libvcpp_attn_gather.so, the same sources
with -DVCPP_GATHER_DUMP) has every decode and prefill kernel record, for each
(sequence or chunk, position) it attends, the physical block and slot its
K/V address was formed from.  The reference gathers position p of a sequence
from block table[p / block_size], slot p % block_size, and skips positions
past the table or whose id is outside the pool (src/paged_attention.cpp:36-42,
src/kv_cache_manager.cpp:90-95).  The dump must equal exactly that: every
attended position recorded with (table[p / BS], p % BS), every skipped or
unattended position left unrecorded.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import DevPool, dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G(cuda):
    return pyvcpp.open_library(pyvcpp.GATHER_LIB_PATH)


def expected(tables, lens, table_lens, nb, bs, stride):
    want = np.full((len(lens), stride, 2), -1, np.int32)
    for s, n in enumerate(lens):
        tl = tables.shape[1] if table_lens is None else min(table_lens[s], tables.shape[1])
        for p in range(int(n)):
            lb = p // bs
            if lb >= tl:
                continue
            bid = int(tables[s, lb])
            if 0 <= bid < nb:
                want[s, p] = (bid, p % bs)
    return want


def run_decode(G, dpool, q, tables, ctx, H, table_lens=None, partition=0):
    stride = int(max(ctx.max(), 1))
    dump = torch.full((len(ctx), stride, 2), -1, dtype=torch.int32, device="cuda:0")
    qd, td, cd = dev(q), dev(tables), dev(ctx)
    tl = None if table_lens is None else dev(table_lens)
    out = torch.empty_like(qd)
    need = G.vcpp_decode_workspace_size(ctypes.byref(dpool.pages), len(ctx), H, int(ctx.max()), partition)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda:0")
    G.vcpp_debug_gather_dump(dump.data_ptr(), stride)
    try:
        rc = G.vcpp_paged_decode(ctypes.byref(dpool.pages), qd.data_ptr(), out.data_ptr(), td.data_ptr(),
                                 tables.shape[1], None if tl is None else tl.data_ptr(), cd.data_ptr(),
                                 len(ctx), int(ctx.max()), H, partition, ws.data_ptr(), ws.numel(), None)
        torch.cuda.synchronize()
    finally:
        G.vcpp_debug_gather_dump(None, 0)
    assert rc == 0, G.vcpp_last_error()
    return dump.cpu().numpy()


def compare(got, want, what):
    bad = np.argwhere(np.any(got != want, axis=-1))
    assert len(bad) == 0, "%s: %d positions differ, first (row, pos) %s: got %s want %s" % (
        what, len(bad), tuple(bad[0]), got[tuple(bad[0])], want[tuple(bad[0])])
    print("%s: %d recorded positions match the block table" % (what, int((want[..., 0] >= 0).sum())))


def tables_for(seed, ctx, nb, bs=16, extra=0):
    nbs = [(int(c) + bs - 1) // bs for c in ctx]
    perm = O.permutation(seed, nb)
    t = np.full((len(ctx), max(max(nbs), 1) + extra), -1, np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    return t


@pytest.mark.parametrize("partition", [0, 64])
def test_decode_config2_gather(G, partition):
    """BASELINE config 2 (64 sequences, ctx U[128, 4096], fp16 pages, random
    tables over a 1.25x pool): page-staged kernel (balanced split) and the
    register-path kernel (64-token partitions)."""
    ctx = O.uniform_int(2024, 64, 128, 4096)
    nb = int(1.25 * sum((int(c) + 15) // 16 for c in ctx))
    pool = O.make_pool(O.ORC_F16, 2025, nb, 8, 80)
    tables = tables_for(2026, ctx, nb)
    q = O.normal(2027, (64, 64, 80))
    got = run_decode(G, DevPool(pool), q, tables, ctx, 64, partition=partition)
    compare(got, expected(tables, ctx, None, nb, 16, got.shape[1]), "config2 P=%d" % partition)


@pytest.mark.parametrize("kind", [O.ORC_F32, O.ORC_F16, O.ORC_I8, O.ORC_FP8])
@pytest.mark.parametrize("partition", [0, 32])
def test_decode_skip_rules_gather(G, kind, partition):
    """Ragged and empty contexts, a short table_lens, ids past the pool and
    negative ids: none of those positions may be loaded."""
    ctx = np.array([0, 1, 15, 16, 17, 100, 257, 700], np.int32)
    nb = 96
    pool = O.make_pool(kind, 77, nb, 8, 80)
    tables = tables_for(78, ctx, nb, extra=2)
    tables[5, 2] = nb + 3
    tables[6, 0] = -5
    tables[7, 10] = nb
    table_lens = np.array([0, 1, 1, 1, 2, 7, 17, 30], np.int32)
    q = O.normal(79, (len(ctx), 64, 80))
    got = run_decode(G, DevPool(pool), q, tables, ctx, 64, table_lens=table_lens, partition=partition)
    compare(got, expected(tables, ctx, table_lens, nb, 16, got.shape[1]),
            "skip rules kind=%d P=%d" % (kind, partition))


def test_decode_block_size_32_gather(G):
    bs, nb = 32, 60
    ctx = np.array([33, 64, 500, 7], np.int32)
    shape = (nb, bs, 8, 80)
    pool = O.Pool(O.ORC_F16, O.f16_trunc(O.normal(81, shape)), O.f16_trunc(O.normal(82, shape)),
                  block_size=bs)
    tables = tables_for(83, ctx, nb, bs=bs)
    got = run_decode(G, DevPool(pool), O.normal(84, (4, 64, 80)), tables, ctx, 64)
    compare(got, expected(tables, ctx, None, nb, bs, got.shape[1]), "block size 32")


def run_prefill(G, dpool, q16, tables, q_start, prefix, H):
    lens = prefix + np.diff(q_start)
    stride = int(lens.max())
    dump = torch.full((len(prefix), stride, 2), -1, dtype=torch.int32, device="cuda:0")
    qd = dev(q16.view(np.uint16))
    out = torch.empty(q16.shape, dtype=torch.float32, device="cuda:0")
    td, qs, pd = dev(tables), dev(q_start), dev(prefix)
    G.vcpp_debug_gather_dump(dump.data_ptr(), stride)
    try:
        rc = G.vcpp_paged_prefill(ctypes.byref(dpool.pages), qd.data_ptr(), out.data_ptr(), td.data_ptr(),
                                  tables.shape[1], qs.data_ptr(), pd.data_ptr(), len(prefix),
                                  int(np.diff(q_start).max()), H, None)
        torch.cuda.synchronize()
    finally:
        G.vcpp_debug_gather_dump(None, 0)
    assert rc == 0, G.vcpp_last_error()
    return dump.cpu().numpy(), lens


def test_prefill_config3_chunk_gather(G):
    """One chunk of BASELINE config 3 (2048 new tokens on a 1024-token paged
    prefix, 64/8 heads, head_dim 80, fp16) plus a second chunk, all tiles."""
    prefix = np.array([1024, 1024], np.int32)
    chunk = np.array([2048, 2048], np.int32)
    lens = prefix + chunk
    nb = int(sum((int(l) + 15) // 16 for l in lens)) + 16
    pool = O.make_pool(O.ORC_F16, 640, nb, 8, 80, 0.0, 0.5)
    tables = tables_for(641, lens, nb)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q16 = O.normal(642, (int(q_start[-1]), 64, 80), 0.0, 0.5).astype(np.float16)
    got, lens = run_prefill(G, DevPool(pool), q16, tables, q_start, prefix, 64)
    compare(got, expected(tables, lens, None, nb, 16, got.shape[1]), "config3 chunks")


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_prefill_skip_rules_gather(G, kind):
    prefix = np.array([45, 0, 130, 300], np.int32)
    chunk = np.array([70, 33, 17, 1], np.int32)
    lens = prefix + chunk
    nb = int(sum((int(l) + 15) // 16 for l in lens)) + 4
    pool = O.make_pool(kind, 650 + kind, nb, 8, 80)
    tables = tables_for(651, lens, nb)
    tables[0, 1] = nb + 2
    tables[2, 5] = -1
    tables[3, 18] = nb
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q16 = O.normal(652, (int(q_start[-1]), 64, 80)).astype(np.float16)
    got, lens = run_prefill(G, DevPool(pool), q16, tables, q_start, prefix, 64)
    compare(got, expected(tables, lens, None, nb, 16, got.shape[1]), "prefill skip rules kind=%d" % kind)
