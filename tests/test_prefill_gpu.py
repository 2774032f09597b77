"""GPU parity of the chunked causal prefill path (vcpp_paged_prefill) against
the CPU oracle's per-position semantics on identical seeded inputs.

Tolerance: max-abs error <= 2e-3 and normwise relative error <= 1e-2 for fp16, int8 and fp8
pages on N(0, 1) data (int8 on the std-2 stress case: 4e-3, see there).
q is fp16 on the GPU; the oracle gets the same fp16 values as fp32.
"""
import os

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import (DevPool, assert_close, gpu_prefill, oracle_prefill_rows, prefill_tables)

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def make_case(kind, seed, prefix, chunk, H, Hkv, D=80, std=1.0, extra_blocks=8):
    lens = [p + n for p, n in zip(prefix, chunk)]
    nb = sum((l + 15) // 16 for l in lens) + extra_blocks
    pool = O.make_pool(kind, seed, nb, Hkv, D, 0.0, std)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q32 = O.normal(seed + 7, (int(q_start[-1]), H, D), 0.0, std)
    q16 = q32.astype(np.float16)
    tables = prefill_tables(seed + 11, lens, nb)
    return pool, q16, q16.astype(np.float32), tables, q_start, np.array(prefix, np.int32)


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
@pytest.mark.parametrize("heads", [(64, 8), (8, 1), (32, 2), (16, 16)])
def test_prefill_small(cuda, kind, heads):
    H, Hkv = heads
    prefix = [0, 19, 1, 64, 200, 0]
    chunk = [1, 21, 64, 65, 37, 130]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 500 + H, prefix, chunk, H, Hkv)
    want = O.prefill(pool, q32, tables, q_start, pre, H)
    got = gpu_prefill(DevPool(pool), q16, tables, q_start, pre, H)
    assert_close(got, want, ATOL, RTOL, what="prefill H=%d Hkv=%d kind=%d" % (H, Hkv, kind))


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
@pytest.mark.parametrize("D", [64, 128])
def test_prefill_head_dims(cuda, D, kind):
    prefix, chunk = [7, 100], [90, 33]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 610 + D, prefix, chunk, 64, 8, D)
    want = O.prefill(pool, q32, tables, q_start, pre, 64)
    got = gpu_prefill(DevPool(pool), q16, tables, q_start, pre, 64)
    assert_close(got, want, ATOL, RTOL, what="prefill D=%d kind=%d" % (D, kind))


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_prefill_skips_invalid_blocks(cuda, kind):
    prefix, chunk = [48, 0], [40, 70]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 620, prefix, chunk, 64, 8)
    tables[0, 1] = -1          # a prefix page missing
    tables[1, 2] = 10 ** 6     # an id past the pool
    want = O.prefill(pool, q32, tables, q_start, pre, 64)
    got = gpu_prefill(DevPool(pool), q16, tables, q_start, pre, 64)
    assert_close(got, want, ATOL, RTOL, what="prefill invalid blocks kind=%d" % kind)


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
@pytest.mark.parametrize("D", [64, 80, 128])
def test_prefill_long_prefix(cuda, kind, D):
    """Prefixes of several hundred 32-key blocks: many trips round the K/V
    ring, odd block counts (a masked tail block), chunk lengths that are not
    multiples of the query tile, and scores large enough (std 2) to move the
    running max many times."""
    prefix, chunk = [2500, 3001, 0], [70, 33, 129]
    pool, q16, q32, tables, q_start, pre = make_case(kind, 650 + D + kind, prefix, chunk, 16, 2,
                                                     D, std=2.0)
    want = O.prefill(pool, q32, tables, q_start, pre, 16)
    got = gpu_prefill(DevPool(pool), q16, tables, q_start, pre, 16)
    # int8 V enters the MFMA as fp16(v * scale): one rounding of at most half
    # an fp16 ulp of the value, so the bound scales with the data (std 2:
    # twice the N(0, 1) bound).  fp16 and FP8 pages hold V exactly.
    atol = ATOL * 2.0 if kind == O.ORC_I8 else ATOL
    assert_close(got, want, atol, RTOL, what="long prefix D=%d kind=%d" % (D, kind))


def test_prefill_matches_decode_for_single_token_chunks(cuda):
    """A chunk of one token on a prefix is a decode step (same oracle row)."""
    prefix, chunk = [300, 17, 1000], [1, 1, 1]
    pool, q16, q32, tables, q_start, pre = make_case(O.ORC_F16, 630, prefix, chunk, 64, 8)
    ctx = pre + 1
    want = O.decode(pool, q32, tables, ctx, 64)
    got = gpu_prefill(DevPool(pool), q16, tables, q_start, pre, 64)
    assert_close(got, want, ATOL, RTOL, what="prefill as decode")


def test_prefill_config3_sampled(cuda):
    """BASELINE config 3 at full size: 8 chunks x 2048 new tokens on 1024-token
    paged prefixes, 64/8 heads, head_dim 80, fp16 N(0, 0.5); all rows run on
    the GPU; 96 random rows (and the first/last of each chunk) and two whole
    chunks are checked."""
    prefix, chunk = [1024] * 8, [2048] * 8
    pool, q16, q32, tables, q_start, pre = make_case(O.ORC_F16, 640, prefix, chunk, 64, 8,
                                                     std=0.5)
    got = gpu_prefill(DevPool(pool), q16, tables, q_start, pre, 64)
    assert np.all(np.isfinite(got))
    rng = np.random.default_rng(7)
    rows = np.unique(np.concatenate([rng.integers(0, q_start[-1], 96), q_start[:-1],
                                     q_start[1:] - 1]))
    want = oracle_prefill_rows(pool, q32, tables, q_start, pre, 64, rows)
    assert_close(got[rows], want, ATOL, RTOL, what="config3 rows")
    # Two whole chunks (the first and the last, 2 x 2048 rows x 64 heads).
    for c in (0, 7):
        r0, r1 = int(q_start[c]), int(q_start[c + 1])
        want_c = O.prefill(pool, q32[r0:r1], tables[c:c + 1], np.array([0, r1 - r0], np.int32),
                           pre[c:c + 1], 64, nthreads=min(16, os.cpu_count() or 1))
        assert_close(got[r0:r1], want_c, ATOL, RTOL, what="config3 whole chunk %d" % c)


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_prefill_block_size_32(cuda, kind):
    """Pages of 32 tokens: a 32-key block is one whole page, and chunk
    boundaries fall inside pages."""
    bs, H, Hkv, D = 32, 16, 2, 80
    prefix, chunk = [45, 0, 130], [70, 33, 17]
    lens = [p + n for p, n in zip(prefix, chunk)]
    nb = sum((l + bs - 1) // bs for l in lens) + 3
    shape = (nb, bs, Hkv, D)
    k = O.normal(301, shape)
    v = O.normal(302, shape)
    if kind == O.ORC_F16:
        pool = O.Pool(kind, O.f16_trunc(k), O.f16_trunc(v), block_size=bs)
    elif kind == O.ORC_FP8:
        pool = O.Pool(kind, O.fp8_encode(k), O.fp8_encode(v), block_size=bs)
    else:
        kq, ks = O.quant_i8(k)
        vq, vs = O.quant_i8(v)
        pool = O.Pool(kind, kq, vq, np.ascontiguousarray(ks.transpose(0, 2, 1)),
                      np.ascontiguousarray(vs.transpose(0, 2, 1)), block_size=bs)
    q_start = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q16 = O.normal(303, (int(q_start[-1]), H, D)).astype(np.float16)
    tables = prefill_tables(304, lens, nb, bs=bs)
    pre = np.array(prefix, np.int32)
    want = O.prefill(pool, q16.astype(np.float32), tables, q_start, pre, H)
    got = gpu_prefill(DevPool(pool), q16.view(np.uint16), tables, q_start, pre, H)
    assert_close(got, want, ATOL, RTOL, what="prefill block_size 32 kind=%d" % kind)
