"""GPU parity of vcpp_write_kv (the device side of KVCacheManager::write_kv,
src/kv_cache_manager.cpp:297-314) against the oracle's encoders: bit-exact
pages for fp32, fp16 (reference truncation, and round-to-nearest on request)
and int8 + fp16 scales; skipped slots leave pages untouched."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import DevPool, dev

pytestmark = pytest.mark.gpu

NB, BS, HKV, D = 12, 16, 4, 80


def special_rows(seed, n):
    x = O.normal(seed, (n, HKV, D), 0.0, 3.0)
    flat = x.reshape(-1)
    sp = np.array([0.0, -0.0, 1 + 3 * 2.0 ** -12, -(1 + 3 * 2.0 ** -12), 6.0e-5, 5.9e-8, -3.0e-8,
                   65504.0, 65520.0, 7.0e4, -1.0e6, 2.0 ** -14, 2.0 ** -15, 1e-3, 0.33333334],
                  np.float32)
    flat[:sp.size] = sp
    x[1] = 0.0          # an all-zero (token, head) row: int8 scale 0
    x[2, 0] *= 1e-6     # tiny row
    return x


def empty_pool(kind):
    shape = (NB, BS, HKV, D)
    if kind == O.ORC_F32:
        return O.Pool(kind, np.full(shape, 7.0, np.float32), np.full(shape, 7.0, np.float32))
    if kind == O.ORC_F16:
        return O.Pool(kind, np.full(shape, 0x1234, np.uint16), np.full(shape, 0x4321, np.uint16))
    if kind == O.ORC_FP8:
        return O.Pool(kind, np.full(shape, 0x5A, np.uint8), np.full(shape, 0xA5, np.uint8))
    sc = np.full((NB, HKV, BS), 0x3C00, np.uint16)
    return O.Pool(kind, np.full(shape, 5, np.int8), np.full(shape, -5, np.int8), sc, sc.copy())


def readback(dp, kind):
    k = dp.k.cpu().numpy()
    v = dp.v.cpu().numpy()
    if kind == O.ORC_F16:
        k, v = k.view(np.uint16), v.view(np.uint16)
    if kind == O.ORC_I8:
        return k, v, dp.ks.cpu().numpy().view(np.uint16), dp.vs.cpu().numpy().view(np.uint16)
    return k, v, None, None


def fp8_rows(seed, n):
    """Rows holding every E4M3 value, every midpoint between neighbours (ties
    go to the smaller code), their float neighbours, and the values past 240
    where the reference's float errors tie across codes (2^32 -> 144, from 2^33
    -> 0)."""
    x = O.normal(seed, (n, HKV, D), 0.0, 30.0).reshape(-1)
    fin = np.sort(O.fp8_decode(np.arange(0x78, dtype=np.uint8)))
    mids = ((fin[1:].astype(np.float64) + fin[:-1]) / 2).astype(np.float32)
    sp = np.concatenate([fin, mids, np.nextafter(mids, np.float32(0)),
                         np.nextafter(mids, np.float32(1e9)),
                         np.array([240.0, 241.0, 300.0, 1e6, 2.0 ** 32, 2.0 ** 33, 1e30, 0.0, -0.0,
                                   np.inf, -np.inf, np.nan, 1e-30, 2.0 ** -10], np.float32)])
    sp = np.concatenate([sp, -sp]).astype(np.float32)
    x[:sp.size] = sp
    return x.reshape(n, HKV, D)


def i8_rows(seed, n):
    """special_rows, plus rows whose int8 quotients x / scale fall exactly on
    half-integers (round half to even decides) and one float either side of
    them: the row max is 127 s so the scale is exactly s, for s = 1/8 and for
    s = fp16(0.1) (their products with k + 1/2 are exact in fp32)."""
    x = special_rows(seed, n)
    for r, sc in ((3, 0.125), (4, float(np.float16(0.1)))):
        for h in range(HKV):
            ks = np.arange(-40, 40, dtype=np.float64)[: D - 1] + 0.5
            ties = (ks * sc).astype(np.float32)
            if h == 1:
                ties = np.nextafter(ties, np.float32(np.inf))
            elif h == 2:
                ties = np.nextafter(ties, np.float32(-np.inf))
            x[r, h, 0] = np.float32(127 * sc)
            x[r, h, 1:] = ties[: D - 1]
    return x


@pytest.mark.parametrize("kind,rne", [(O.ORC_F32, 0), (O.ORC_F16, 0), (O.ORC_F16, 1), (O.ORC_I8, 0),
                                      (O.ORC_FP8, 0)])
def test_write_kv_bit_exact(cuda, kind, rne):
    n = 40
    rows = fp8_rows if kind == O.ORC_FP8 else i8_rows if kind == O.ORC_I8 else special_rows
    k = rows(71, n)
    v = rows(72, n)
    slots = O.permutation(73, NB * BS)[:n].astype(np.int64)
    slots[5] = -1                 # skipped
    slots[6] = NB * BS + 3        # block past the pool: skipped
    pool = empty_pool(kind)
    dp = DevPool(pool)
    pyvcpp.write_kv(dp.pages, dev(k), dev(v), dev(slots), fp16_round_nearest=bool(rne))
    torch.cuda.synchronize()
    gk, gv, gks, gvs = readback(dp, kind)
    wk, wv = pool.k.copy(), pool.v.copy()
    wks = None if pool.k_scale is None else pool.k_scale.copy()
    wvs = None if pool.v_scale is None else pool.v_scale.copy()
    for t in range(n):
        s = int(slots[t])
        if s < 0 or s >= NB * BS:
            continue
        b, p = divmod(s, BS)
        for src, dst, sdst in ((k[t], wk, wks), (v[t], wv, wvs)):
            if kind == O.ORC_F32:
                dst[b, p] = src
            elif kind == O.ORC_F16:
                dst[b, p] = src.astype(np.float16).view(np.uint16) if rne else O.f16_trunc(src)
            elif kind == O.ORC_FP8:
                dst[b, p] = O.fp8_encode(src)
            else:
                q, sc = O.quant_i8(src)
                dst[b, p] = q
                sdst[b, :, p] = sc
    np.testing.assert_array_equal(gk, wk)
    np.testing.assert_array_equal(gv, wv)
    if kind == O.ORC_I8:
        np.testing.assert_array_equal(gks, wks)
        np.testing.assert_array_equal(gvs, wvs)


@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_write_then_prefill(cuda, kind):
    """Pages written on the device from fp32 K/V, then a causal prefill over
    them, equal the oracle on pages the oracle encoded itself."""
    from gpu_util import assert_close, gpu_prefill
    H, Hkv, Dd = 16, 2, 80
    lens = [150, 37]
    nb = 24
    k = O.normal(81, (sum(lens), Hkv, Dd))
    v = O.normal(82, (sum(lens), Hkv, Dd))
    tables = O.permutation(83, nb)[:20].reshape(2, 10).astype(np.int32)
    slots = np.concatenate([tables[i, np.arange(n) // 16] * 16 + np.arange(n) % 16
                            for i, n in enumerate(lens)]).astype(np.int64)
    shape = (nb, 16, Hkv, Dd)
    if kind == O.ORC_F16:
        host = O.Pool(kind, np.zeros(shape, np.uint16), np.zeros(shape, np.uint16))
    elif kind == O.ORC_FP8:
        host = O.Pool(kind, np.zeros(shape, np.uint8), np.zeros(shape, np.uint8))
    else:
        host = O.Pool(kind, np.zeros(shape, np.int8), np.zeros(shape, np.int8),
                      np.zeros((nb, Hkv, 16), np.uint16), np.zeros((nb, Hkv, 16), np.uint16))
    dp = DevPool(host)
    pyvcpp.write_kv(dp.pages, dev(k), dev(v), dev(slots))
    torch.cuda.synchronize()
    gk, gv, gks, gvs = readback(dp, kind)
    # oracle pages from the same rows
    for t, s in enumerate(slots):
        b, p = divmod(int(s), 16)
        if kind == O.ORC_F16:
            host.k[b, p], host.v[b, p] = O.f16_trunc(k[t]), O.f16_trunc(v[t])
        elif kind == O.ORC_FP8:
            host.k[b, p], host.v[b, p] = O.fp8_encode(k[t]), O.fp8_encode(v[t])
        else:
            (host.k[b, p], host.k_scale[b, :, p]), (host.v[b, p], host.v_scale[b, :, p]) = \
                O.quant_i8(k[t]), O.quant_i8(v[t])
    np.testing.assert_array_equal(gk, host.k)
    np.testing.assert_array_equal(gv, host.v)
    q_start = np.array([0, 50, 60], np.int32)
    prefix = np.array([lens[0] - 50, lens[1] - 10], np.int32)
    q32 = O.normal(84, (60, H, Dd))
    q16 = q32.astype(np.float16)
    want = O.prefill(host, q16.astype(np.float32), tables, q_start, prefix, H)
    got = gpu_prefill(dp, q16.view(np.uint16), tables, q_start, prefix, H)
    assert_close(got, want, 2e-3, 1e-2, what="write then prefill kind=%d" % kind)


@pytest.mark.parametrize("d", [10, 16, 24, 40, 64, 128])
@pytest.mark.parametrize("kind", [O.ORC_F16, O.ORC_I8, O.ORC_FP8])
def test_write_kv_head_dims(cuda, kind, d):
    """Head dims that pick each writer: 10 (not a multiple of 4) the
    one-wave-per-row kernel; 24 and 40 eight values per lane on an odd lane
    count per row for fp16 / FP8, four per lane for int8; 16, 64, 128 eight
    per lane on an even lane count."""
    nb, bs, hkv, n = 6, 16, 3, 50
    x = O.normal(91 + d, (n, hkv, d), 0.0, 4.0)
    y = O.normal(92 + d, (n, hkv, d), 0.0, 4.0)
    x[3, 1] *= 1e-6  # a tiny row next to ordinary ones
    slots = O.permutation(93, nb * bs)[:n].astype(np.int64)
    shape = (nb, bs, hkv, d)
    if kind == O.ORC_F16:
        host = O.Pool(kind, np.zeros(shape, np.uint16), np.zeros(shape, np.uint16))
    elif kind == O.ORC_FP8:
        host = O.Pool(kind, np.zeros(shape, np.uint8), np.zeros(shape, np.uint8))
    else:
        host = O.Pool(kind, np.zeros(shape, np.int8), np.zeros(shape, np.int8),
                      np.zeros((nb, hkv, bs), np.uint16), np.zeros((nb, hkv, bs), np.uint16))
    dp = DevPool(host)
    pyvcpp.write_kv(dp.pages, dev(x), dev(y), dev(slots))
    torch.cuda.synchronize()
    gk, gv, gks, gvs = readback(dp, kind)
    for t, s in enumerate(slots):
        b, p = divmod(int(s), bs)
        for src, dst, sdst in ((x[t], host.k, host.k_scale), (y[t], host.v, host.v_scale)):
            if kind == O.ORC_F16:
                dst[b, p] = O.f16_trunc(src)
            elif kind == O.ORC_FP8:
                dst[b, p] = O.fp8_encode(src)
            else:
                q, sc = O.quant_i8(src)
                dst[b, p] = q
                sdst[b, :, p] = sc
    np.testing.assert_array_equal(gk, host.k)
    np.testing.assert_array_equal(gv, host.v)
    if kind == O.ORC_I8:
        np.testing.assert_array_equal(gks, host.k_scale)
        np.testing.assert_array_equal(gvs, host.v_scale)
