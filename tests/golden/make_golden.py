"""Writes tests/golden/golden_vectors.npz from the compiled reference.

Run in the build container, where oracle/_ref/libref.so is built from the
reference's own src/paged_attention.cpp, src/kv_cache_manager.cpp and
src/quantization.cpp (oracle/Makefile).  Inputs come from the oracle's
seeded splitmix64/Box-Muller generator; the fixture stores the outputs plus
a checksum of every input so a generator drift is caught, not masked.

    python tests/golden/make_golden.py
"""
import os
import sys
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

OUT = os.path.join(HERE, "golden_vectors.npz")


def crc(*arrays):
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).tobytes(), c)
    return np.uint32(c)


def table_for(seed, ctx, num_blocks):
    nbs = [(c + O.BS - 1) // O.BS for c in ctx]
    mb = max(max(nbs), 1)
    perm = O.permutation(seed, num_blocks)
    t = np.full((len(ctx), mb), -1, dtype=np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    return t


def main():
    assert O.ref_available(), "oracle/_ref/libref.so missing: run `make -C oracle`"
    out = {}

    # Config 1: 1 seq, ctx 512, 64/8 heads, D 80, 32 logical blocks drawn from a
    # random permutation of 64 physical blocks; FP32 pool.
    k = O.normal(101, (64, 16, 8, 80))
    v = O.normal(102, (64, 16, 8, 80))
    q = O.normal(103, (1, 64, 80))
    table = O.permutation(107, 64)[:32].reshape(1, 32)
    ctx = np.array([512], dtype=np.int32)
    ref = O.RefPool(k, v, fp16=False)
    out["config1_out"] = ref.decode(q, table, ctx, 64)
    out["config1_crc"] = crc(k, v, q, table)

    # The same inputs through the reference FP16 pool (truncating encoder).
    ref16 = O.RefPool(k, v, fp16=True)
    rk, rv = ref16.raw()
    out["config1_f16_out"] = ref16.decode(q, table, ctx, 64)
    out["config1_f16_kcrc"] = crc(rk, rv)

    # Tiny cases: ctx in {0,1,15,16,17,33} for H/Hkv in {1/1, 8/1, 64/8}, both pools.
    ctxs = np.array([0, 1, 15, 16, 17, 33], dtype=np.int32)
    for H, Hkv in ((1, 1), (8, 1), (64, 8)):
        nb = 24
        k = O.normal(200 + H, (nb, 16, Hkv, 80))
        v = O.normal(300 + H, (nb, 16, Hkv, 80))
        q = O.normal(400 + H, (len(ctxs), H, 80))
        t = table_for(500 + H, ctxs, nb)
        for fp16 in (False, True):
            r = O.RefPool(k, v, fp16=fp16)
            key = "tiny_h%d_kv%d_%s" % (H, Hkv, "f16" if fp16 else "f32")
            out[key] = r.decode(q, t, ctxs, H)
        out["tiny_h%d_kv%d_crc" % (H, Hkv)] = crc(k, v, q, t)

    # Chunked prefill with the engine's per-position causal semantics:
    # chunk 0 = 21 new tokens on a 19-token prefix, chunk 1 = 7 tokens, no prefix.
    H, Hkv, nb = 16, 2, 24
    k = O.normal(601, (nb, 16, Hkv, 80))
    v = O.normal(602, (nb, 16, Hkv, 80))
    prefix = np.array([19, 0], dtype=np.int32)
    q_start = np.array([0, 21, 28], dtype=np.int32)
    q = O.normal(603, (28, H, 80))
    lens = [19 + 21, 7]
    t = table_for(604, lens, nb)
    r = O.RefPool(k, v, fp16=True)
    out["prefill_out"] = r.prefill(q, t, q_start, prefix, H)
    out["prefill_crc"] = crc(k, v, q, t)

    # fp16 encoder known answers through KVCacheManager::write_kv.
    specials = np.array([1 + 3 * 2 ** -12, -1 - 3 * 2 ** -12, 65504.0, 65520.0, 1e6, -1e6,
                         2 ** -14, 2 ** -15, 1e-8, -0.0, 0.0, np.inf, -np.inf, np.nan,
                         0.1, -0.3333333, 3.14159265, 2 ** -14 * 1.5], dtype=np.float32)
    kk = np.zeros((1, 16, 1, 80), dtype=np.float32)
    kk.reshape(-1)[:len(specials)] = specials
    r = O.RefPool(kk, kk, fp16=True)
    rk, _ = r.raw()
    out["f16_specials_in"] = specials
    out["f16_specials_bits"] = rk.reshape(-1)[:len(specials)].copy()

    np.savez_compressed(OUT, **out)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
