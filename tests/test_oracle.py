"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: the committed golden vectors from the compiled reference, the live
compiled reference (oracle/_ref, when built), numpy's IEEE fp16 conversion,
closed forms, fp64 brute force and the split-K identity.
"""
import os

import numpy as np
import pytest

import oracle_lib as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_vectors.npz")
BS = O.BS


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def crc(*arrays):
    import zlib
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).tobytes(), c)
    return np.uint32(c)


def tables_for(seed, ctx, nb):
    nbs = [(c + BS - 1) // BS for c in ctx]
    mb = max(max(nbs), 1)
    perm = O.permutation(seed, nb)
    t = np.full((len(ctx), mb), -1, dtype=np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    return t


# ---- golden vectors (compiled reference, committed) -------------------------

def test_golden_config1(gold):
    k = O.normal(101, (64, 16, 8, 80))
    v = O.normal(102, (64, 16, 8, 80))
    q = O.normal(103, (1, 64, 80))
    table = O.permutation(107, 64)[:32].reshape(1, 32)
    assert crc(k, v, q, table) == gold["config1_crc"], "input generator drifted"
    ctx = np.array([512], dtype=np.int32)
    out = O.decode(O.Pool(O.ORC_F32, k, v), q, table, ctx, 64)
    np.testing.assert_allclose(out, gold["config1_out"], atol=1e-6, rtol=1e-5)
    # FP16 pool: the oracle's truncating encoder reproduces the reference pool bits.
    kh, vh = O.f16_trunc(k), O.f16_trunc(v)
    assert crc(kh, vh) == gold["config1_f16_kcrc"]
    out16 = O.decode(O.Pool(O.ORC_F16, kh, vh), q, table, ctx, 64)
    np.testing.assert_allclose(out16, gold["config1_f16_out"], atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("H,Hkv", [(1, 1), (8, 1), (64, 8)])
def test_golden_tiny(gold, H, Hkv):
    ctxs = np.array([0, 1, 15, 16, 17, 33], dtype=np.int32)
    nb = 24
    k = O.normal(200 + H, (nb, 16, Hkv, 80))
    v = O.normal(300 + H, (nb, 16, Hkv, 80))
    q = O.normal(400 + H, (len(ctxs), H, 80))
    t = tables_for(500 + H, ctxs, nb)
    assert crc(k, v, q, t) == gold["tiny_h%d_kv%d_crc" % (H, Hkv)]
    for name, pool in (("f32", O.Pool(O.ORC_F32, k, v)),
                       ("f16", O.Pool(O.ORC_F16, O.f16_trunc(k), O.f16_trunc(v)))):
        out = O.decode(pool, q, t, ctxs, H)
        np.testing.assert_allclose(out, gold["tiny_h%d_kv%d_%s" % (H, Hkv, name)],
                                   atol=1e-6, rtol=1e-5)
        assert np.all(out[0] == 0.0)


def test_golden_prefill(gold):
    H, Hkv, nb = 16, 2, 24
    k = O.normal(601, (nb, 16, Hkv, 80))
    v = O.normal(602, (nb, 16, Hkv, 80))
    prefix = np.array([19, 0], dtype=np.int32)
    q_start = np.array([0, 21, 28], dtype=np.int32)
    q = O.normal(603, (28, H, 80))
    t = tables_for(604, [40, 7], nb)
    assert crc(k, v, q, t) == gold["prefill_crc"]
    pool = O.Pool(O.ORC_F16, O.f16_trunc(k), O.f16_trunc(v))
    out = O.prefill(pool, q, t, q_start, prefix, H)
    np.testing.assert_allclose(out, gold["prefill_out"], atol=1e-6, rtol=1e-5)


def test_golden_f16_specials(gold):
    bits = O.f16_trunc(gold["f16_specials_in"])
    assert np.array_equal(bits, gold["f16_specials_bits"])
    # Truncation, not rounding: 1 + 3*2^-12 -> 0x3C00 (RNE would give 0x3C01).
    assert O.orc().orc_f16_encode_trunc(1 + 3 * 2 ** -12) == 0x3C00


# ---- live compiled reference ------------------------------------------------

@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("fp16", [False, True])
def test_live_reference_decode(fp16):
    nb, H, Hkv = 40, 32, 4
    ctx = np.array([1, 50, 200, 333], dtype=np.int32)
    k = O.normal(901, (nb, 16, Hkv, 80), 0.3, 2.0)
    v = O.normal(902, (nb, 16, Hkv, 80), -0.1, 0.5)
    q = O.normal(903, (4, H, 80))
    t = tables_for(904, ctx, nb)
    t[2, 1] = 10 ** 6  # invalid id: skipped by both
    ref = O.RefPool(k, v, fp16=fp16)
    want = ref.decode(q, t, ctx, H)
    pool = O.Pool(O.ORC_F16, *ref.raw()) if fp16 else O.Pool(O.ORC_F32, k, v)
    got = O.decode(pool, q, t, ctx, H)
    np.testing.assert_allclose(got, want, atol=1e-6, rtol=1e-5)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_live_reference_short_table():
    """seq_len beyond the table: the reference skips those positions."""
    nb, H, Hkv = 16, 8, 1
    k = O.normal(911, (nb, 16, Hkv, 80))
    v = O.normal(912, (nb, 16, Hkv, 80))
    q = O.normal(913, (2, H, 80))
    t = np.array([[3, 5], [7, 1]], dtype=np.int32)
    ctx = np.array([100, 20], dtype=np.int32)
    ref = O.RefPool(k, v, fp16=False)
    np.testing.assert_allclose(O.decode(O.Pool(O.ORC_F32, k, v), q, t, ctx, H),
                               ref.decode(q, t, ctx, H), atol=1e-6, rtol=1e-5)


# ---- closed forms and brute force ------------------------------------------

def test_ctx1_returns_v_row():
    pool = O.make_pool(O.ORC_F32, 1, 4, 2, 80)
    q = O.normal(2, (1, 8, 80))
    t = np.array([[3]], dtype=np.int32)
    out = O.decode(pool, q, t, np.array([1], np.int32), 8)
    for h in range(8):
        np.testing.assert_array_equal(out[0, h], pool.v[3, 0, h // 4])


def test_constant_keys_give_mean_of_v():
    nb, Hkv = 4, 1
    k = np.ones((nb, 16, Hkv, 80), np.float32) * 0.25
    v = O.normal(5, (nb, 16, Hkv, 80))
    pool = O.Pool(O.ORC_F32, k, v)
    q = O.normal(6, (1, 4, 80))
    t = np.array([[2, 0, 3]], dtype=np.int32)
    ctx = 40
    out = O.decode(pool, q, t, np.array([ctx], np.int32), 4)
    rows = np.concatenate([v[2, :, 0], v[0, :, 0], v[3, :8, 0]])
    np.testing.assert_allclose(out[0], np.broadcast_to(rows.mean(0), (4, 80)), atol=2e-6)


def test_dominant_logit_selects_row():
    nb, Hkv = 2, 1
    k = O.normal(7, (nb, 16, Hkv, 80)) * 0.01
    k[1, 5, 0] = 0.0
    k[1, 5, 0, 0] = 1000.0
    v = O.normal(8, (nb, 16, Hkv, 80))
    q = np.zeros((1, 1, 80), np.float32)
    q[0, 0, 0] = 1.0
    out = O.decode(O.Pool(O.ORC_F32, k, v), q, np.array([[0, 1]], np.int32),
                   np.array([32], np.int32), 1)
    np.testing.assert_allclose(out[0, 0], v[1, 5, 0], atol=1e-6)


def test_group_heads_with_equal_q_agree():
    pool = O.make_pool(O.ORC_F16, 9, 8, 2, 80)
    q1 = O.normal(10, (1, 1, 80))
    q = np.repeat(q1, 16, axis=1)
    out = O.decode(pool, q, np.array([[1, 2, 3]], np.int32), np.array([45], np.int32), 16)
    for h in range(8):
        np.testing.assert_array_equal(out[0, h], out[0, 0])
        np.testing.assert_array_equal(out[0, 8 + h], out[0, 8])


def test_brute_force_fp64():
    nb, Hkv, H, D = 6, 2, 4, 80
    pool = O.make_pool(O.ORC_F32, 12, nb, Hkv, D)
    q = O.normal(13, (1, H, D))
    t = np.array([[4, 1, 5, 0]], dtype=np.int32)
    ctx = 53
    out = O.decode(pool, q, t, np.array([ctx], np.int32), H)
    for h in range(H):
        kvh = h // (H // Hkv)
        ks = np.stack([pool.k[t[0, p // 16], p % 16, kvh] for p in range(ctx)]).astype(np.float64)
        vs = np.stack([pool.v[t[0, p // 16], p % 16, kvh] for p in range(ctx)]).astype(np.float64)
        s = ks @ q[0, h].astype(np.float64) / np.sqrt(D)
        w = np.exp(s - s.max())
        want = (w / w.sum()) @ vs
        np.testing.assert_allclose(out[0, h], want, atol=2e-6, rtol=1e-5)
        # the C fp64 brute force agrees too
        o64 = np.empty(D, np.float64)
        O.orc().orc_dense_f64(O._p(q[0, h].astype(np.float64)), O._p(np.ascontiguousarray(ks)),
                              O._p(np.ascontiguousarray(vs)), ctx, D, 1 / np.sqrt(D), O._p(o64))
        np.testing.assert_allclose(o64, want, atol=1e-12)


def test_split_k_identity():
    import ctypes
    pool = O.make_pool(O.ORC_F16, 14, 40, 1, 80)
    q = O.normal(15, (1, 1, 80))
    t = np.arange(40, dtype=np.int32)[::-1].copy()
    ctx = 600
    whole = O.single(pool, q[0], t, ctx, 1)[0]
    s = pool.orc_struct()
    P = 96
    parts = [(p0, min(p0 + P, ctx)) for p0 in range(0, ctx, P)]
    m = np.empty(len(parts), np.float32)
    l = np.empty(len(parts), np.float32)
    o = np.empty((len(parts), 80), np.float32)
    for i, (a, b) in enumerate(parts):
        O.orc().orc_partial(ctypes.byref(s), O._p(q[0, 0]), 0, O._p(t), len(t), a, b,
                            O._p(m[i:i + 1]), O._p(l[i:i + 1]), O._p(o[i]))
    merged = np.empty(80, np.float32)
    O.orc().orc_lse_merge(O._p(m), O._p(l), O._p(o), len(parts), 80, O._p(merged))
    np.testing.assert_allclose(merged, whole, atol=1e-6, rtol=1e-5)


def test_block_permutation_invariance():
    """Moving pages to other physical blocks (same logical order) is bit-identical."""
    pool = O.make_pool(O.ORC_F32, 16, 10, 2, 80)
    q = O.normal(17, (1, 8, 80))
    t = np.array([[1, 4, 7]], dtype=np.int32)
    a = O.decode(pool, q, t, np.array([40], np.int32), 8)
    perm = np.array([9, 8, 7, 6, 5, 4, 3, 2, 1, 0])
    k2 = np.empty_like(pool.k)
    v2 = np.empty_like(pool.v)
    k2[perm] = pool.k
    v2[perm] = pool.v
    b = O.decode(O.Pool(O.ORC_F32, k2, v2), q, perm[t].astype(np.int32), np.array([40], np.int32), 8)
    np.testing.assert_array_equal(a, b)


# ---- codecs ------------------------------------------------------------------

def test_f16_decode_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_decode(bits)
    want = bits.view(np.float16).astype(np.float32)
    exp31 = ((bits >> 10) & 0x1F) == 31
    np.testing.assert_array_equal(got[~exp31], want[~exp31])
    # the reference maps exponent 31 (inf and NaN alike) to +/-inf
    assert np.all(np.isinf(got[exp31]))
    assert np.all(np.signbit(got[exp31]) == ((bits[exp31] >> 15) == 1))


def test_f16_rne_matches_numpy():
    x = np.concatenate([O.normal(18, (20000,), 0, 3), O.normal(19, (2000,), 0, 1e-5),
                        np.array([65504, 65519, 65520, 1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                                  0.0, -0.0], np.float32)]).astype(np.float32)
    got = np.array([O.orc().orc_f16_encode_rne(float(v)) for v in x], dtype=np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_quant_i8_known_answers():
    x = np.zeros((1, 80), np.float32)
    x[0, :3] = [1.0, -0.5, 0.25]
    q, s = O.quant_i8(x)
    assert s[0] == 0x2008  # fp16(1/127) = 0.0078735...
    assert list(q[0, :4]) == [127, -64, 32, 0]
    q0, s0 = O.quant_i8(np.zeros((1, 80), np.float32))
    assert s0[0] == 0 and not q0.any()
    # reconstruction error is at most half a step (plus the fp16 scale rounding)
    y = O.normal(20, (64, 80))
    q, s = O.quant_i8(y)
    sc = O.f16_decode(s)[:, None]
    assert np.all(np.abs(q.astype(np.float32) * sc - y) <= 0.5 * sc * 1.01 + 1e-7)
    assert np.abs(q).max() == 127


def test_generator_statistics():
    x = O.normal(21, (200000,))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    a = O.normal(21, (1000,))
    np.testing.assert_array_equal(a, x[:1000])  # index-stable stream
    p = O.permutation(22, 1000)
    assert sorted(p) == list(range(1000))
    u = O.uniform_int(23, 10000, 128, 4096)
    assert u.min() >= 128 and u.max() <= 4096


def test_flash_attention_brute_force():
    """orc_flash_attention (cuda/attention.cu:58-124) against a float64 dense
    softmax of query row 0; rows 1.. of q never matter."""
    B, H, ql, kv, D = 2, 3, 4, 37, 80
    q = O.normal(901, (B, H, ql, D))
    k = O.normal(902, (B, H, kv, D))
    v = O.normal(903, (B, H, kv, D))
    out, w = O.flash(q, k, v)
    for b in range(B):
        for h in range(H):
            s = k[b, h].astype(np.float64) @ q[b, h, 0].astype(np.float64) / np.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            np.testing.assert_allclose(w[b * H + h], p, atol=1e-6, rtol=1e-5)
            np.testing.assert_allclose(out[b, h], p @ v[b, h].astype(np.float64), atol=2e-6, rtol=1e-5)
    q2 = q.copy()
    q2[:, :, 1:] = 123.0
    out2, _ = O.flash(q2, k, v)
    np.testing.assert_array_equal(out2, out)


def test_flash_attention_mask():
    """attn_mask[s] < 0 sets logit s to -1e9: with one position left open the
    output is that V row and its weight is 1."""
    B, H, kv, D = 1, 2, 9, 16
    q = O.normal(911, (B, H, 1, D))
    k = O.normal(912, (B, H, kv, D))
    v = O.normal(913, (B, H, kv, D))
    mask = -np.ones(kv, np.float32)
    mask[5] = 0.0
    out, w = O.flash(q, k, v, mask)
    for h in range(H):
        np.testing.assert_allclose(out[0, h], v[0, h, 5], atol=1e-6)
        assert abs(w[h, 5] - 1.0) < 1e-6 and np.all(w[h, np.arange(kv) != 5] == 0.0)


# ---- FP8 E4M3 pages (src/quantization.cpp, the reference's KV_FP8 pool) ----

def test_fp8_decode_known_values():
    # bias 7, 3 mantissa bits; 0x77 = 1.875 * 2^7 = 240; exponent 15 = inf/NaN
    known = {0x00: 0.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9, 0x08: 2.0 ** -6, 0x38: 1.0,
             0x39: 1.125, 0x3F: 1.875, 0x40: 2.0, 0x77: 240.0, 0xB8: -1.0, 0xF7: -240.0}
    for b, v in known.items():
        assert O.fp8_decode(np.array([b], np.uint8))[0] == np.float32(v), hex(b)
    sp = O.fp8_decode(np.array([0x7E, 0xFE, 0x7F, 0xFF, 0x78, 0x7D], np.uint8))
    assert sp[0] == np.inf and sp[1] == -np.inf and np.all(np.isnan(sp[2:]))


def test_fp8_encode_known_answers():
    x = np.array([1.0, 1.0625, 1.0625001, 1.1875, 240.0, 250.0, 2.0 ** 32, 2.0 ** 34, 1e30,
                  np.inf, -np.inf, np.nan, -0.0, 0.0, 2.0 ** -10, 2.0 ** -10 * 1.0001,
                  3 * 2.0 ** -10, -1.5, 0.015625, -1e30], np.float32)
    want = [0x38,
            0x38,  # 1.0625: halfway between 1.0 and 1.125, the first (smaller) code wins
            0x39,
            0x39,  # 1.1875: halfway between 1.125 and 1.25
            0x77, 0x77,  # saturate at 240
            0x71,  # 2^32: fl(a - v) is the same for v in [144, 240], the first such code wins
            0x00, 0x00,  # from 2^33, fl(a - v) == a for every code: code 0 wins
            0x7E, 0xFE, 0xFF,
            0x00,  # -0.0: the write path takes the sign from v < 0
            0x00, 0x00, 0x01, 0x01, 0xBC, 0x08,
            0x80]  # the first code of the negative half is -0
    got = O.fp8_encode(x)
    assert [hex(v) for v in got] == [hex(v) for v in want]


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_fp8_codec_matches_reference():
    """Every code decodes as the reference pool decodes it; the encoder agrees
    with the reference's write path on every code's value, every midpoint
    between neighbours (the tie rule), their float neighbours, specials and a
    log-uniform sweep."""
    L = O.ref()
    codes = np.arange(256, dtype=np.uint8)
    want = np.empty(256, np.float32)
    L.ref_fp8_decode_n(O._p(codes), O._p(want), 256)
    np.testing.assert_array_equal(O.fp8_decode(codes), want)
    fin = np.sort(want[np.isfinite(want) & (want >= 0)])
    mids = ((fin[1:].astype(np.float64) + fin[:-1]) / 2).astype(np.float32)
    xs = np.concatenate([fin, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                         np.array([245.0, 248.0, 256.0, 1e10, 2.0 ** 32, 2.0 ** 33, 2.0 ** 33 + 2048,
                                   2.0 ** -12, 1e-30, 0.0, np.inf, np.nan], np.float32),
                         np.exp(np.random.default_rng(1).uniform(-12, 7, 20000)).astype(np.float32)])
    xs = np.concatenate([xs, -xs]).astype(np.float32)
    ref_b = np.empty(xs.shape, np.uint8)
    L.ref_fp8_encode_n(O._p(xs), O._p(ref_b), xs.size)
    np.testing.assert_array_equal(O.fp8_encode(xs), ref_b)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_fp8_pool_attention_matches_reference():
    """The reference's own FP8_E4M3 pool (write_kv encodes, get_k decodes)
    against the oracle's FP8 pool: identical pages, identical outputs."""
    nb, hkv, D, H = 40, 8, 80, 64
    k = O.normal(71, (nb, O.BS, hkv, D), std=2.0)
    v = O.normal(72, (nb, O.BS, hkv, D), std=2.0)
    rp = O.RefPool(k, v, fp8=True)
    rk, rv = rp.raw()
    pool = O.make_pool(O.ORC_FP8, 71, nb, hkv, D, std=2.0)
    np.testing.assert_array_equal(pool.k, rk)
    np.testing.assert_array_equal(pool.v, rv)
    ctx = np.array([1, 17, 100, 200], np.int32)
    perm = O.permutation(73, nb)
    tables = np.full((4, 13), -1, np.int32)
    off = 0
    for i, c in enumerate(ctx):
        n = (c + O.BS - 1) // O.BS
        tables[i, :n] = perm[off:off + n]
        off += n
    q = O.normal(74, (4, H, D))
    # the reference build contracts to FMA (see test_live_reference_decode)
    np.testing.assert_allclose(O.decode(pool, q, tables, ctx, H), rp.decode(q, tables, ctx, H),
                               atol=1e-6, rtol=1e-5)
