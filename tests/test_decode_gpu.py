"""GPU parity of the paged decode path (vcpp_paged_decode / paged_attention_cuda)
against the CPU oracle on identical seeded inputs.

Tolerances (max-abs error <= atol, and normwise relative error <= rtol):
  fp32 KV: atol 1e-4, rtol 1e-4;  fp16 / int8 / fp8 KV: atol 2e-3, rtol 1e-2.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import DevPool, assert_close, dev, gpu_decode

pytestmark = pytest.mark.gpu

TOL = {O.ORC_F32: (1e-4, 1e-4), O.ORC_F16: (2e-3, 1e-2), O.ORC_I8: (2e-3, 1e-2),
       O.ORC_FP8: (2e-3, 1e-2)}
KINDS = [O.ORC_F32, O.ORC_F16, O.ORC_I8, O.ORC_FP8]


def random_tables(seed, ctx, num_blocks, max_blocks=None):
    nbs = [(c + O.BS - 1) // O.BS for c in ctx]
    mb = max(max(nbs), 1) if max_blocks is None else max_blocks
    perm = O.permutation(seed, num_blocks)
    t = np.full((len(ctx), mb), -1, dtype=np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    assert k <= num_blocks
    return t


def config1(kind=O.ORC_F32):
    """1 seq, ctx 512, 64/8 heads, D 80, 32 logical blocks on
    a random permutation of 64 physical blocks, N(0,1)."""
    pool = O.make_pool(kind, 101, 64, 8, 80)
    q = O.normal(103, (1, 64, 80))
    table = O.permutation(107, 64)[:32].reshape(1, 32)
    return pool, q, table, np.array([512], dtype=np.int32)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("partition", [0, 64, 512])
def test_config1(cuda, kind, partition):
    pool, q, table, ctx = config1(kind)
    want = O.decode(pool, q, table, ctx, 64)
    got = gpu_decode(DevPool(pool), q, table, ctx, 64, partition_size=partition)
    assert_close(got, want, *TOL[kind], what="config1 kind=%d P=%d" % (kind, partition))


@pytest.mark.parametrize("partition", [64, 0])
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("heads", [(1, 1), (8, 1), (64, 8), (12, 4), (32, 2), (32, 8), (24, 8),
                                   (8, 8), (56, 8)])
def test_small_cases(cuda, kind, heads, partition):
    H, Hkv = heads
    ctx = np.array([0, 1, 15, 16, 17, 33, 100, 257], dtype=np.int32)
    nb = 64
    pool = O.make_pool(kind, 11 + H, nb, Hkv, 80)
    q = O.normal(13 + H, (len(ctx), H, 80))
    tables = random_tables(17, ctx, nb)
    want = O.decode(pool, q, tables, ctx, H)
    got = gpu_decode(DevPool(pool), q, tables, ctx, H, partition_size=partition)
    assert_close(got, want, *TOL[kind], what="small H=%d Hkv=%d kind=%d P=%d" % (H, Hkv, kind, partition))
    assert np.all(got[0] == 0.0), "ctx=0 must give zeros"


@pytest.mark.parametrize("partition", [128, 0])
@pytest.mark.parametrize("D", [64, 128])
def test_other_head_dims(cuda, D, partition):
    ctx = np.array([5, 48, 300], dtype=np.int32)
    pool = O.make_pool(O.ORC_F16, 21, 40, 8, D)
    q = O.normal(23, (3, 64, D))
    tables = random_tables(29, ctx, 40)
    want = O.decode(pool, q, tables, ctx, 64)
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64, partition_size=partition)
    assert_close(got, want, *TOL[O.ORC_F16], what="D=%d P=%d" % (D, partition))


@pytest.mark.parametrize("partition", [64, 0])
@pytest.mark.parametrize("kind", KINDS)
def test_skip_rules(cuda, kind, partition):
    """Invalid block ids and positions past the table are skipped, as the
    reference does (src/paged_attention.cpp:38,42)."""
    nb = 48
    pool = O.make_pool(kind, 31, nb, 8, 80)
    ctx = np.array([200, 200, 200, 64], dtype=np.int32)
    q = O.normal(37, (4, 64, 80))
    tables = random_tables(41, ctx, nb)
    tables[0, 3] = -5          # negative id
    tables[1, 7] = nb + 100    # id past the pool
    table_lens = np.array([13, 13, 6, 2], dtype=np.int32)  # row 2/3 shorter than ctx
    want = O.decode(pool, q, tables, ctx, 64, table_lens=table_lens)
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64, table_lens=table_lens,
                     partition_size=partition)
    assert_close(got, want, *TOL[kind], what="skip rules kind=%d P=%d" % (kind, partition))


def test_all_positions_skipped_gives_zero(cuda):
    pool = O.make_pool(O.ORC_F16, 43, 8, 8, 80)
    ctx = np.array([40, 40], dtype=np.int32)
    q = O.normal(47, (2, 64, 80))
    tables = np.full((2, 3), -1, dtype=np.int32)
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64, partition_size=32)
    assert np.all(got == 0.0)


def test_split_invariance(cuda):
    """The same sequences with every partition size agree with the oracle."""
    nb = 600
    pool = O.make_pool(O.ORC_F16, 53, nb, 8, 80)
    ctx = np.array([4000, 1, 777, 2048, 33], dtype=np.int32)
    q = O.normal(59, (5, 64, 80))
    tables = random_tables(61, ctx, nb)
    want = O.decode(pool, q, tables, ctx, 64)
    dp = DevPool(pool)
    outs = []
    for P in (32, 96, 256, 1024):
        got = gpu_decode(dp, q, tables, ctx, 64, partition_size=P)
        assert_close(got, want, *TOL[O.ORC_F16], what="P=%d" % P)
        outs.append(got)
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) < 1e-4


def test_config2_full(cuda):
    """BASELINE config 2 at full size: 64 seqs, ctx U[128,4096], fp16 pages in a
    pool of 1.25x the tokens, random tables; every output checked."""
    ctx = O.uniform_int(71, 64, 128, 4096)
    nb = int(np.ceil(1.25 * ctx.sum() / O.BS))
    pool = O.make_pool(O.ORC_F16, 73, nb, 8, 80)
    q = O.normal(79, (64, 64, 80))
    tables = random_tables(83, ctx, nb)
    want = O.decode(pool, q, tables, ctx, 64)
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64)
    assert_close(got, want, *TOL[O.ORC_F16], what="config2")


def test_v1_entry(cuda):
    """paged_attention_cuda (cuda/attention.h:19-30) on the v1 layout
    [nb][2][BS][Hkv][D] with host context_lens."""
    nb = 80
    pool = O.make_pool(O.ORC_F16, 89, nb, 8, 80)
    ctx = np.array([300, 5, 129], dtype=np.int32)
    q = O.normal(97, (3, 64, 80))
    tables = random_tables(101, ctx, nb)
    want = O.decode(pool, q, tables, ctx, 64)
    kv = np.stack([pool.k, pool.v], axis=1)  # [nb][2][BS][Hkv][D]
    kvd = dev(kv)
    qd = dev(q)
    out = torch.zeros_like(qd)
    td = dev(tables)
    L = pyvcpp.lib()
    L.paged_attention_cuda(qd.data_ptr(), kvd.data_ptr(), td.data_ptr(), ctx.ctypes.data,
                           out.data_ptr(), 64, 8, 80, 16, 3)
    torch.cuda.synchronize()
    assert pyvcpp.last_error() == ""
    assert_close(out.cpu().numpy(), want, *TOL[O.ORC_F16], what="v1")


def _allocation_end(ptr):
    """End address of the device allocation holding ptr (hipMemGetAddressRange)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    base, size = ctypes.c_void_p(), ctypes.c_size_t()
    rc = hip.hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), ctypes.c_void_p(ptr))
    assert rc == 0 and base.value, "hipMemGetAddressRange failed (%d)" % rc
    return base.value + size.value


def test_v1_skips_ids_past_the_allocation(cuda):
    """v1 carries no block count: block ids whose page would end past the
    allocation that holds kv_cache are skipped, as the reference's get_k skips
    ids outside the pool (src/kv_cache_manager.cpp:90-95)."""
    nb = 40
    pool = O.make_pool(O.ORC_F16, 91, nb, 8, 80)
    ctx = np.array([200, 64], dtype=np.int32)
    q = O.normal(93, (2, 64, 80))
    tables = random_tables(95, ctx, nb)
    kv = np.stack([pool.k, pool.v], axis=1)
    kvd = dev(kv)
    block_bytes = 2 * 16 * 8 * 80 * 2
    past = (_allocation_end(kvd.data_ptr()) - kvd.data_ptr()) // block_bytes
    assert past >= nb
    bad = tables.copy()
    bad[0, 3] = past          # first id whose page ends past the allocation
    bad[1, 1] = past + 1000
    # The oracle skips ids >= num_blocks; give it the same skips.
    want_tables = tables.copy()
    want_tables[0, 3] = nb + 5
    want_tables[1, 1] = nb + 5
    want = O.decode(pool, q, want_tables, ctx, 64)
    qd = dev(q)
    out = torch.zeros_like(qd)
    L = pyvcpp.lib()
    L.paged_attention_cuda(qd.data_ptr(), kvd.data_ptr(), dev(bad).data_ptr(), ctx.ctypes.data,
                           out.data_ptr(), 64, 8, 80, 16, 2)
    torch.cuda.synchronize()
    assert pyvcpp.last_error() == ""
    assert_close(out.cpu().numpy(), want, *TOL[O.ORC_F16], what="v1 ids past the allocation")


@pytest.mark.parametrize("partition", [0, 32, 128])
def test_workspace_reuse(cuda, partition):
    """One workspace across many calls with changing q and pages: no call may
    see a previous call's partials."""
    nb = 400
    pools = [O.make_pool(O.ORC_F16, 300 + i, nb, 8, 80) for i in range(2)]
    dpools = [DevPool(pl) for pl in pools]
    ctx = np.array([1500, 40, 777, 16, 2900, 0, 129, 700], dtype=np.int32)
    tables = random_tables(311, ctx, nb)
    td, cd = dev(tables), dev(ctx)
    need = pyvcpp.decode_workspace_size(dpools[0].pages, len(ctx), 64, int(ctx.max()), partition)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda:0")
    for it in range(6):
        q = O.normal(400 + it, (len(ctx), 64, 80))
        want = O.decode(pools[it % 2], q, tables, ctx, 64)
        qd = dev(q)
        out = torch.full_like(qd, float("nan"))
        pyvcpp.paged_decode(dpools[it % 2].pages, qd, out, td, cd, int(ctx.max()), 64,
                            partition_size=partition, workspace=ws)
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), want, *TOL[O.ORC_F16], what="reuse it=%d" % it)


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_many_short_sequences(cuda, kind):
    """Hundreds of short, ragged sequences (many per workgroup range, several
    empty) and a few long ones that span several ranges: the balanced split
    (which charges every sequence start) switches sequence inside ranges
    constantly, over several 64-sequence scan steps."""
    rng = np.random.default_rng(3)
    ctx = rng.integers(0, 70, 700).astype(np.int32)
    ctx[::37] = 0
    ctx[[5, 300, 301, 650]] = [3000, 2500, 40, 4096]
    nb = int(sum((c + 15) // 16 for c in ctx)) + 16
    pool = O.make_pool(kind, 211, nb, 8, 80)
    q = O.normal(212, (len(ctx), 64, 80))
    tables = random_tables(213, ctx, nb)
    want = O.decode(pool, q, tables, ctx, 64)
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64)
    assert_close(got, want, *TOL[kind], what="many short kind=%d" % kind)
    assert np.all(got[ctx == 0] == 0.0)


def test_block_size_32(cuda):
    """Pages of 32 tokens: a 16-token tile is half a page."""
    bs = 32
    ctx = np.array([1000, 31, 64, 33, 0, 500], dtype=np.int32)
    nbs = [(c + bs - 1) // bs for c in ctx]
    nb = sum(nbs) + 5
    shape = (nb, bs, 8, 80)
    k = O.f16_trunc(O.normal(221, shape))
    v = O.f16_trunc(O.normal(222, shape))
    perm = O.permutation(223, nb)
    tables = np.full((len(ctx), max(nbs)), -1, np.int32)
    o = 0
    for i, n in enumerate(nbs):
        tables[i, :n] = perm[o:o + n]
        o += n
    q = O.normal(224, (len(ctx), 64, 80))
    pool = O.Pool(O.ORC_F16, k, v, block_size=bs)
    # the oracle's pool struct carries the block size of its pages
    want = O.decode(pool, q, tables, ctx, 64)
    dp = DevPool(pool)
    got = gpu_decode(dp, q, tables, ctx, 64)
    assert_close(got, want, *TOL[O.ORC_F16], what="block size 32")


@pytest.mark.parametrize("partition", [0, 128])
@pytest.mark.parametrize("D", [64, 128])
def test_fp8_other_head_dims(cuda, D, partition):
    """FP8 pages (the reference KV_FP8 pool's E4M3 bytes) on the page-staged
    kernel (D 64) and the register-path kernel (D 128, fixed partitions)."""
    ctx = np.array([5, 48, 300, 1], dtype=np.int32)
    pool = O.make_pool(O.ORC_FP8, 231, 40, 8, D, std=3.0)
    q = O.normal(233, (4, 64, D))
    tables = random_tables(239, ctx, 40)
    want = O.decode(pool, q, tables, ctx, 64)
    got = gpu_decode(DevPool(pool), q, tables, ctx, 64, partition_size=partition)
    assert_close(got, want, *TOL[O.ORC_FP8], what="fp8 D=%d P=%d" % (D, partition))


@pytest.mark.parametrize("partition", [0, 64])
@pytest.mark.parametrize("D", [64, 80, 128])
@pytest.mark.parametrize("heads", [(64, 8), (32, 4), (16, 4), (24, 8)])
@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_page_kernel_shapes(cuda, kind, heads, D, partition):
    """Every page-staged kernel shape (8 kv heads per workgroup at head_dim 64
    and 80; 4 per workgroup for 4-head multiples and head_dim 128, walked as
    head groups of one range) on ragged contexts, both split modes."""
    H, Hkv = heads
    ctx = np.array([0, 5, 16, 31, 300, 1025, 777, 64, 2000, 1], dtype=np.int32)
    nb = int(sum((int(c) + O.BS - 1) // O.BS for c in ctx)) + 6
    pool = O.make_pool(kind, 3000 + D + H, nb, Hkv, D)
    q = O.normal(3100 + D + H, (len(ctx), H, D))
    tables = random_tables(3200 + D, ctx, nb)
    want = O.decode(pool, q, tables, ctx, H)
    got = gpu_decode(DevPool(pool), q, tables, ctx, H, partition_size=partition)
    assert_close(got, want, *TOL[kind], what="page shapes kind=%d H=%d Hkv=%d D=%d P=%d"
                 % (kind, H, Hkv, D, partition))
    assert np.all(got[0] == 0.0), "ctx=0 must give zeros"
