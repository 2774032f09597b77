"""Exact properties of the paged decode and prefill paths at BASELINE's full
sizes, where the CPU oracle would take minutes; every check is bit-for-bit
(torch.equal).

- Physical block placement: moving every page to another physical block and
  rewriting the tables to match leaves the output unchanged.  The kernels walk
  positions in logical order, so only values, never addresses, enter the
  arithmetic (the reference's `table[p / 16]`, slot `p % 16` indexing,
  src/paged_attention.cpp:36-37).
- GQA sharing: query heads of one kv group given the same q get the same
  output (each head's softmax and P V run on its own MFMA rows).
- V doubling (fp16 pages): V times 2 is exact in fp16, P does not depend on V,
  and fp32 products and sums scale by 2 exactly, so the output doubles.

Inputs are generated on the device (torch generators, fixed seeds): config 2
is 64 sequences with ctx ~ U[128, 4096] over a pool of 1.25x the blocks,
config 3 is 8 chunks of 2048 new tokens on 1024-token paged prefixes; 64 q /
8 kv heads, head_dim 80, pages of 16 tokens."""
import numpy as np
import pytest
import torch

import pyvcpp

pytestmark = pytest.mark.gpu

H, HKV, D, BS = 64, 8, 80, 16


def _gen(seed):
    return torch.Generator(device="cuda:0").manual_seed(seed)


def make_pages(kind, nb, seed):
    """Random K/V pages [nb][BS][HKV][D] (+ int8 scales [nb][HKV][BS])."""
    g = _gen(seed)
    shape = (nb, BS, HKV, D)
    ks = vs = None
    if kind == pyvcpp.KV_F16:
        k = torch.randn(shape, generator=g, device="cuda:0").half().view(torch.int16)
        v = torch.randn(shape, generator=g, device="cuda:0").half().view(torch.int16)
    elif kind == pyvcpp.KV_I8:
        k = torch.randint(-127, 128, shape, generator=g, device="cuda:0", dtype=torch.int8)
        v = torch.randint(-127, 128, shape, generator=g, device="cuda:0", dtype=torch.int8)
        sc = (nb, HKV, BS)
        ks = (torch.rand(sc, generator=g, device="cuda:0") * 0.01 + 0.005).half().view(torch.int16)
        vs = (torch.rand(sc, generator=g, device="cuda:0") * 0.01 + 0.005).half().view(torch.int16)
    else:  # FP8 E4M3 codes with exponent field < 15 (finite values, |x| < 256)
        def codes():
            b = torch.randint(0, 256, shape, generator=g, device="cuda:0", dtype=torch.int32)
            b = torch.where((b & 0x78) == 0x78, b & 0xF7, b)  # exponent 15 -> 14
            return b.to(torch.uint8)
        k, v = codes(), codes()
    return k, v, ks, vs


def pages_desc(kind, k, v, ks, vs):
    nb = k.shape[0]
    return pyvcpp.kv_pages(kind, k, v, BS, HKV, D, nb, BS * HKV * D, ks, vs, HKV * BS)


def config2_tables(seed, ctx, nb):
    nbs = (ctx + BS - 1) // BS
    perm = np.random.default_rng(seed).permutation(nb).astype(np.int32)
    tables = np.full((64, int(nbs.max())), -1, np.int32)
    o = 0
    for i, n in enumerate(nbs):
        tables[i, :n] = perm[o:o + n]
        o += n
    return tables


def move_blocks(k, v, ks, vs, tables, seed):
    """The same pages at other physical blocks: block b moves to pi[b]."""
    nb = k.shape[0]
    pi = torch.from_numpy(np.random.default_rng(seed).permutation(nb)).to("cuda:0")
    def moved(x):
        if x is None:
            return None
        y = torch.empty_like(x)
        y[pi] = x
        return y
    t = torch.from_numpy(tables).to("cuda:0").long()
    t2 = torch.where(t >= 0, pi[t.clamp(min=0)], t).to(torch.int32)
    return moved(k), moved(v), moved(ks), moved(vs), t2


def decode(desc, q, tables, ctx):
    out = torch.full_like(q, float("nan"))
    pyvcpp.paged_decode(desc, q, out, tables, torch.from_numpy(ctx).to("cuda:0"),
                        int(ctx.max()), H)
    torch.cuda.synchronize()
    return out


@pytest.fixture(scope="module")
def config2_shape():
    ctx = np.random.default_rng(900).integers(128, 4097, 64).astype(np.int32)
    nb = int(np.ceil(1.25 * ctx.sum() / BS))
    return ctx, config2_tables(901, ctx, nb), nb


@pytest.mark.parametrize("kind", [pyvcpp.KV_F16, pyvcpp.KV_I8, pyvcpp.KV_FP8])
def test_decode_config2_block_placement(cuda, config2_shape, kind):
    ctx, tables, nb = config2_shape
    k, v, ks, vs = make_pages(kind, nb, 901 + kind)
    q = torch.randn((64, H, D), generator=_gen(905), device="cuda:0")
    a = decode(pages_desc(kind, k, v, ks, vs), q, torch.from_numpy(tables).to("cuda:0"), ctx)
    k2, v2, ks2, vs2, t2 = move_blocks(k, v, ks, vs, tables, 906)
    b = decode(pages_desc(kind, k2, v2, ks2, vs2), q, t2, ctx)
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("kind", [pyvcpp.KV_F16, pyvcpp.KV_I8, pyvcpp.KV_FP8])
def test_decode_config2_gqa_equal_queries(cuda, config2_shape, kind):
    ctx, tables, nb = config2_shape
    k, v, ks, vs = make_pages(kind, nb, 911 + kind)
    q = torch.randn((64, HKV, 1, D), generator=_gen(915), device="cuda:0")
    q = q.expand(64, HKV, H // HKV, D).reshape(64, H, D).contiguous()
    out = decode(pages_desc(kind, k, v, ks, vs), q, torch.from_numpy(tables).to("cuda:0"), ctx)
    assert torch.isfinite(out).all()
    grouped = out.view(64, HKV, H // HKV, D)
    assert torch.equal(grouped, grouped[:, :, :1].expand_as(grouped))


def test_decode_config2_v_doubling(cuda, config2_shape):
    ctx, tables, nb = config2_shape
    k, v, _, _ = make_pages(pyvcpp.KV_F16, nb, 921)
    q = torch.randn((64, H, D), generator=_gen(925), device="cuda:0")
    t = torch.from_numpy(tables).to("cuda:0")
    a = decode(pages_desc(pyvcpp.KV_F16, k, v, None, None), q, t, ctx)
    v2 = (v.view(torch.float16) * 2).view(torch.int16)
    b = decode(pages_desc(pyvcpp.KV_F16, k, v2, None, None), q, t, ctx)
    assert torch.isfinite(a).all()
    assert torch.equal(b, a * 2)


# ---- prefill, BASELINE config 3 -------------------------------------------------

PREFIX, CHUNK, NCHUNK = 1024, 2048, 8


@pytest.fixture(scope="module")
def config3_case():
    lens = [PREFIX + CHUNK] * NCHUNK
    nbs = [(n + BS - 1) // BS for n in lens]
    nb = sum(nbs) + 16
    rng = np.random.default_rng(930)
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((NCHUNK, max(nbs)), -1, np.int32)
    o = 0
    for i, n in enumerate(nbs):
        tables[i, :n] = perm[o:o + n]
        o += n
    g = _gen(931)
    shape = (nb, BS, HKV, D)
    k = (torch.randn(shape, generator=g, device="cuda:0") * 0.5).half().view(torch.int16)
    v = (torch.randn(shape, generator=g, device="cuda:0") * 0.5).half().view(torch.int16)
    q = (torch.randn((NCHUNK * CHUNK, H, D), generator=g, device="cuda:0") * 0.5).half()
    q_start = torch.arange(0, (NCHUNK + 1) * CHUNK, CHUNK, dtype=torch.int32, device="cuda:0")
    prefix = torch.full((NCHUNK,), PREFIX, dtype=torch.int32, device="cuda:0")
    return k, v, q, tables, q_start, prefix


def prefill(k, v, q, tables, q_start, prefix):
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    pyvcpp.paged_prefill(pages_desc(pyvcpp.KV_F16, k, v, None, None), q.view(torch.int16), out,
                         tables, q_start, prefix, CHUNK, H)
    torch.cuda.synchronize()
    return out


def test_prefill_config3_block_placement(cuda, config3_case):
    k, v, q, tables, q_start, prefix = config3_case
    a = prefill(k, v, q, torch.from_numpy(tables).to("cuda:0"), q_start, prefix)
    k2, v2, _, _, t2 = move_blocks(k, v, None, None, tables, 932)
    b = prefill(k2, v2, q, t2, q_start, prefix)
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)


def test_prefill_config3_v_doubling(cuda, config3_case):
    k, v, q, tables, q_start, prefix = config3_case
    t = torch.from_numpy(tables).to("cuda:0")
    a = prefill(k, v, q, t, q_start, prefix)
    v2 = (v.view(torch.float16) * 2).view(torch.int16)
    b = prefill(k, v2, q, t, q_start, prefix)
    assert torch.equal(b, a * 2)


def test_prefill_config3_gqa_equal_queries(cuda, config3_case):
    k, v, q, tables, q_start, prefix = config3_case
    n = q.shape[0]
    qg = q.view(n, HKV, H // HKV, D)[:, :, :1].expand(n, HKV, H // HKV, D).reshape(n, H, D).contiguous()
    out = prefill(k, v, qg, torch.from_numpy(tables).to("cuda:0"), q_start, prefix)
    assert torch.isfinite(out).all()
    grouped = out.view(n, HKV, H // HKV, D)
    assert torch.equal(grouped, grouped[:, :, :1].expand_as(grouped))
