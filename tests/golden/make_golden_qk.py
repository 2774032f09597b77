"""Writes tests/golden/golden_qk.npz from the compiled reference engine helpers.

Run in the build container, where oracle/_ref/libref_engine.so is built from
the reference's own src/paged_engine.cpp (and the sources it links with) by
oracle/Makefile.  It records rope_single (src/paged_engine.cpp:47-62) and the
engine's rms_norm (:14-20) on seeded inputs: the outputs, the positions, and a
checksum of every input (regenerated from the oracle's seeded generator).

    python tests/golden/make_golden_qk.py
"""
import os
import sys

import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

OUT = os.path.join(HERE, "golden_qk.npz")


def crc(*arrays):
    c = 0
    for a in arrays:
        c = zlib.crc32(np.ascontiguousarray(a).tobytes(), c)
    return np.uint32(c)

# (head_dim, heads, positions, inv_freq size or 0 = full table)
ROPE_CASES = [(80, 8, [0, 1, 17, 511, 4095, 32767], 0),
              (128, 2, [3, 100000], 0),
              (64, 4, [5, 999], 7)]  # short table: the min(i, size - 1) clamp


def rope_inputs(i, hd, heads, npos, nf):
    x = O.normal(9100 + i, (npos, heads * hd))
    f = O.inv_freq_table(hd)
    if nf:
        f = f[:nf].copy()
    return x, f


def main():
    L = O.ref_engine()
    out = {}
    for i, (hd, heads, pos, nf) in enumerate(ROPE_CASES):
        x, f = rope_inputs(i, hd, heads, len(pos), nf)
        y = x.copy()
        for t, p in enumerate(pos):
            row = y[t]  # contiguous view
            L.ref_rope_single(O._p(row), heads * hd, hd, p, O._p(f), len(f))
        out[f"rope{i}_pos"] = np.array(pos, np.int32)
        out[f"rope{i}_crc"] = crc(x, f)
        out[f"rope{i}_out"] = y
    for i, (hd, eps) in enumerate([(80, 1e-6), (128, 1e-5)]):
        x = O.normal(9200 + i, (16, hd), std=3.0)
        w = O.normal(9300 + i, (hd,), mean=1.0, std=0.1)
        y = np.zeros_like(x)
        for r in range(x.shape[0]):
            L.ref_rms_norm(O._p(x[r]), O._p(w), O._p(y[r]), hd, eps)
        out[f"norm{i}_crc"] = crc(x, w)
        out[f"norm{i}_eps"] = np.float32(eps)
        out[f"norm{i}_out"] = y
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
