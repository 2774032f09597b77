"""Seeded random shapes for decode and prefill against the CPU oracle: page
dtypes, head dims, GQA groupings, page sizes, split modes and ragged or empty
contexts drawn together, so that combinations the hand-written cases do not
name are covered too.  Tolerances as in the other parity tests (numpy allclose
form, err <= atol + rtol * |want|): fp32 pages 1e-4 / 1e-4, fp16 / int8 / FP8
pages 2e-3 / 1e-2."""
import numpy as np
import pytest

import oracle_lib as O
from gpu_util import DevPool, assert_close, gpu_decode, gpu_prefill, gpu_prefill_split, prefill_tables

pytestmark = pytest.mark.gpu

TOL = {O.ORC_F32: (1e-4, 1e-4), O.ORC_F16: (2e-3, 1e-2), O.ORC_I8: (2e-3, 1e-2),
       O.ORC_FP8: (2e-3, 1e-2)}
HEADS = [(64, 8), (8, 1), (32, 4), (16, 16), (24, 8)]


def tables_for(rng, ctx, nb, bs):
    nbs = [(int(c) + bs - 1) // bs for c in ctx]
    perm = rng.permutation(nb).astype(np.int32)
    t = np.full((len(ctx), max(max(nbs), 1)), -1, np.int32)
    o = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[o:o + n]
        o += n
    return t


def pool_for(kind, seed, nb, hkv, d, bs):
    if bs == 16:
        return O.make_pool(kind, seed, nb, hkv, d)
    shape = (nb, bs, hkv, d)  # fp16 pages of another size
    return O.Pool(O.ORC_F16, O.f16_trunc(O.normal(seed, shape)), O.f16_trunc(O.normal(seed + 1, shape)),
                  block_size=bs)


@pytest.mark.parametrize("case", range(16))
def test_decode_random(cuda, case):
    rng = np.random.default_rng(7000 + case)
    kind = int(rng.choice([O.ORC_F32, O.ORC_F16, O.ORC_I8, O.ORC_FP8]))
    H, Hkv = HEADS[int(rng.integers(len(HEADS)))]
    D = int(rng.choice([64, 80, 128]))
    bs = 32 if kind == O.ORC_F16 and rng.random() < 0.3 else 16
    partition = int(rng.choice([0, 0, 64, 256]))
    n = int(rng.integers(1, 24))
    ctx = rng.integers(0, 1600, n).astype(np.int32)
    ctx[rng.random(n) < 0.15] = 0
    ctx[rng.random(n) < 0.15] = rng.integers(1, 20)
    nb = int(sum((int(c) + bs - 1) // bs for c in ctx)) + 4
    print("decode case %d: kind %d H %d Hkv %d D %d bs %d partition %d seqs %d tokens %d"
          % (case, kind, H, Hkv, D, bs, partition, n, int(ctx.sum())), flush=True)
    pool = pool_for(kind, 7100 + case, nb, Hkv, D, bs)
    q = O.normal(7200 + case, (n, H, D))
    tables = tables_for(rng, ctx, nb, bs)
    want = O.decode(pool, q, tables, ctx, H)
    got = gpu_decode(DevPool(pool), q, tables, ctx, H, partition_size=partition)
    assert_close(got, want, *TOL[kind], what="decode case %d" % case)


@pytest.mark.parametrize("case", range(10))
def test_prefill_random(cuda, case):
    rng = np.random.default_rng(8000 + case)
    kind = int(rng.choice([O.ORC_F16, O.ORC_I8, O.ORC_FP8]))
    H, Hkv = HEADS[int(rng.integers(len(HEADS)))]
    D = int(rng.choice([64, 80, 128]))
    nc = int(rng.integers(1, 6))
    prefix = rng.integers(0, 500, nc).astype(np.int32)
    prefix[rng.random(nc) < 0.3] = 0
    chunk = rng.integers(1, 150, nc).astype(np.int32)
    lens = [int(p + c) for p, c in zip(prefix, chunk)]
    nb = sum((l + 15) // 16 for l in lens) + 4
    print("prefill case %d: kind %d H %d Hkv %d D %d chunks %s prefixes %s"
          % (case, kind, H, Hkv, D, list(chunk), list(prefix)), flush=True)
    pool = O.make_pool(kind, 8100 + case, nb, Hkv, D)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q32 = O.normal(8200 + case, (int(q_start[-1]), H, D))
    q16 = q32.astype(np.float16)
    tables = prefill_tables(8300 + case, lens, nb)
    want = O.prefill(pool, q16.astype(np.float32), tables, q_start, prefix, H)
    got = gpu_prefill(DevPool(pool), q16.view(np.uint16), tables, q_start, prefix, H)
    assert_close(got, want, *TOL[kind], what="prefill case %d" % case)


@pytest.mark.parametrize("case", range(8))
def test_prefill_split_random(cuda, case):
    """vcpp_paged_prefill_split on few chunks with long, ragged prefixes (the
    shapes it splits) and some it leaves unsplit."""
    rng = np.random.default_rng(8500 + case)
    kind = int(rng.choice([O.ORC_F16, O.ORC_I8, O.ORC_FP8]))
    H, Hkv = HEADS[int(rng.integers(len(HEADS)))]
    D = int(rng.choice([64, 80, 128]))
    nc = int(rng.integers(1, 4))
    prefix = rng.integers(0, 5000, nc).astype(np.int32)
    prefix[rng.random(nc) < 0.2] = 0
    chunk = rng.integers(0, 200, nc).astype(np.int32)
    chunk[0] = max(int(chunk[0]), 1)
    lens = [int(p + c) for p, c in zip(prefix, chunk)]
    nb = sum((l + 15) // 16 for l in lens) + 4
    print("split prefill case %d: kind %d H %d Hkv %d D %d chunks %s prefixes %s"
          % (case, kind, H, Hkv, D, list(chunk), list(prefix)), flush=True)
    pool = O.make_pool(kind, 8600 + case, nb, Hkv, D)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q16 = O.normal(8700 + case, (int(q_start[-1]), H, D)).astype(np.float16)
    tables = prefill_tables(8800 + case, lens, nb)
    want = O.prefill(pool, q16.astype(np.float32), tables, q_start, prefix, H)
    got, split = gpu_prefill_split(DevPool(pool), q16.view(np.uint16), tables, q_start, prefix, H)
    print("  split: %s" % split, flush=True)
    assert_close(got, want, *TOL[kind], what="split prefill case %d" % case)
