"""CPU pins of the oracle's query/key preparation: per-head RMS norm and RoPE.

- golden fixtures written by the compiled reference (tests/golden/golden_qk.npz,
  from rope_single and rms_norm of src/paged_engine.cpp);
- a live comparison with oracle/_ref/libref_engine.so where it is built;
- closed forms and invariants that a dropped term, a swapped sign or a wrong
  pairing would break: position 0 is the identity, a rotation keeps every pair's
  length, complex multiplication by e^{i theta} in float64, the relative-position
  identity <R(a) q, R(b) k> = <R(a - c) q, R(b - c) k>, and the index permutation
  that maps the interleaved pairing onto the half-split one;
- hand-computed known answers for apply_rope_cuda's partner clamp.
"""
import os

import numpy as np
import pytest

import oracle_lib as O
from golden.make_golden_qk import ROPE_CASES, crc, rope_inputs

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_qk.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


@pytest.mark.parametrize("i", range(len(ROPE_CASES)))
def test_rope_matches_reference_golden(gold, i):
    hd, heads, pos, nf = ROPE_CASES[i]
    x, f = rope_inputs(i, hd, heads, len(pos), nf)
    assert crc(x, f) == gold[f"rope{i}_crc"], "input generator drifted"
    y = O.rope(x.reshape(len(pos), heads, hd), pos, f, O.ROPE_INTERLEAVED)
    np.testing.assert_array_equal(y.reshape(len(pos), -1), gold[f"rope{i}_out"])


@pytest.mark.parametrize("i,hd", [(0, 80), (1, 128)])
def test_head_norm_matches_reference_golden(gold, i, hd):
    x = O.normal(9200 + i, (16, hd), std=3.0)
    w = O.normal(9300 + i, (hd,), mean=1.0, std=0.1)
    assert crc(x, w) == gold[f"norm{i}_crc"]
    y = O.head_norm(x, w, float(gold[f"norm{i}_eps"]))
    np.testing.assert_array_equal(y, gold[f"norm{i}_out"])


@pytest.mark.skipif(not O.ref_engine_available(), reason="oracle/_ref not built")
def test_rope_live_reference_many_positions():
    hd, heads = 80, 8
    rng = np.random.default_rng(5)
    pos = rng.integers(0, 40000, 64).astype(np.int32)
    x = rng.standard_normal((64, heads * hd)).astype(np.float32)
    f = O.inv_freq_table(hd)
    want = x.copy()
    for t in range(64):
        O.ref_engine().ref_rope_single(O._p(want[t]), heads * hd, hd, int(pos[t]), O._p(f), len(f))
    got = O.rope(x.reshape(64, heads, hd), pos, f, O.ROPE_INTERLEAVED).reshape(64, -1)
    np.testing.assert_array_equal(got, want)


def test_rope_position_zero_is_identity():
    x = O.normal(1, (3, 4, 80))
    for style in (O.ROPE_INTERLEAVED, O.ROPE_HALF):
        np.testing.assert_array_equal(O.rope(x, [0, 0, 0], O.inv_freq_table(80), style), x)


def pairs(x, style):
    D = x.shape[-1]
    if style == O.ROPE_INTERLEAVED:
        return x[..., 0::2], x[..., 1::2]
    return x[..., : D // 2], x[..., D // 2:]


@pytest.mark.parametrize("style", [O.ROPE_INTERLEAVED, O.ROPE_HALF])
def test_rope_is_complex_rotation(style):
    D = 80
    x = O.normal(2, (5, 3, D))
    pos = np.array([1, 7, 100, 2048, 30000], np.int32)
    f = O.inv_freq_table(D)
    y = O.rope(x, pos, f, style)
    a, b = pairs(x.astype(np.float64), style)
    theta = (f[None, :] * pos[:, None].astype(np.float32)).astype(np.float64)  # fp32 product
    z = (a + 1j * b) * np.exp(1j * theta)[:, None, :]
    ya, yb = pairs(y.astype(np.float64), style)
    np.testing.assert_allclose(ya, z.real, atol=2e-6, rtol=0)
    np.testing.assert_allclose(yb, z.imag, atol=2e-6, rtol=0)
    # lengths of the pairs are kept
    np.testing.assert_allclose(np.hypot(ya, yb), np.hypot(a, b), rtol=1e-6)


def test_rope_relative_position_identity():
    D = 64
    f = O.inv_freq_table(D, base=10000.0)
    q = O.normal(3, (1, 1, D))
    k = O.normal(4, (1, 1, D))
    for a, b, c in [(10, 3, 2), (50, 50, 20), (7, 30, 5)]:
        lhs = float(np.dot(O.rope(q, [a], f, 0).ravel(), O.rope(k, [b], f, 0).ravel()))
        rhs = float(np.dot(O.rope(q, [a - c], f, 0).ravel(), O.rope(k, [b - c], f, 0).ravel()))
        assert abs(lhs - rhs) < 1e-4 * (1 + abs(lhs))


def test_rope_styles_related_by_permutation():
    D = 80
    x = O.normal(6, (4, 2, D))
    pos = [3, 9, 333, 4000]
    f = O.inv_freq_table(D)
    perm = np.concatenate([np.arange(0, D, 2), np.arange(1, D, 2)])  # interleaved -> half layout
    half = O.rope(x[..., perm], pos, f, O.ROPE_HALF)
    inter = O.rope(x, pos, f, O.ROPE_INTERLEAVED)
    np.testing.assert_array_equal(half, inter[..., perm])


def test_rope_short_table_clamps_to_last_frequency():
    D = 16
    f = np.array([1.0, 0.5, 0.25], np.float32)
    x = O.normal(7, (1, 1, D))
    y = O.rope(x, [3], f, O.ROPE_INTERLEAVED)
    full = np.array([1.0, 0.5] + [0.25] * 6, np.float32)
    np.testing.assert_array_equal(y, O.rope(x, [3], full, O.ROPE_INTERLEAVED))


def test_head_norm_closed_forms():
    D = 80
    x = O.normal(8, (6, D), std=2.0)
    w = np.ones(D, np.float32)
    y = O.head_norm(x, w, 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1)), 1.0, rtol=1e-6)
    # scale invariance without eps, the weight multiplies elementwise
    np.testing.assert_allclose(O.head_norm(4.0 * x, w, 0.0), y, rtol=1e-6, atol=1e-7)
    w2 = O.normal(9, (D,), mean=1.0, std=0.2)
    np.testing.assert_allclose(O.head_norm(x, w2, 0.0), y * w2, rtol=2e-6, atol=1e-7)
    # float64 statement with eps
    x64 = x.astype(np.float64)
    want = w2 * x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + 1e-2)
    np.testing.assert_allclose(O.head_norm(x, w2, 1e-2), want, rtol=2e-6)
    # zero row: eps keeps it finite, output zero
    z = O.head_norm(np.zeros((1, D), np.float32), w2, 1e-6)
    assert np.all(z == 0)


def test_rope_table_known_answers():
    # head_dim 4, total_dim 6: head 0 pairs (0,2),(1,3); head 1 holds d 4, 5 with
    # hdim 0, 1 < 2 -> partners 6, 7 past total_dim -> clamped to themselves, so
    # the kept value is x s + x c.
    cs = np.array([0.5, 0.25], np.float32)
    sn = np.array([0.75, -1.0], np.float32)
    q = np.array([[1, 2, 3, 4, 5, 6]], np.float32)
    k = -q
    qo, ko = O.rope_table(q, k, cs, sn, 4)
    want = np.array([[1 * 0.5 - 3 * 0.75, 2 * 0.25 - 4 * -1.0, 1 * 0.75 + 3 * 0.5, 2 * -1.0 + 4 * 0.25,
                      5 * 0.75 + 5 * 0.5, 6 * -1.0 + 6 * 0.25]], np.float32)
    np.testing.assert_array_equal(qo, want)
    np.testing.assert_array_equal(ko, -want)


def test_rope_table_equals_half_style_at_one_position():
    D, H, pos = 80, 3, 1234
    f = O.inv_freq_table(D)
    theta = f * np.float32(pos)
    cs = np.cos(theta).astype(np.float32)
    sn = np.sin(theta).astype(np.float32)
    x = O.normal(10, (2, H * D))
    qo, _ = O.rope_table(x, x, cs, sn, D)
    # the half-split rotation with the same cos/sin values (computed by the
    # oracle's cosf/sinf at the same fp32 angle) agrees to fp32 rounding
    y = O.rope(x.reshape(2, H, D), [pos, pos], f, O.ROPE_HALF).reshape(2, -1)
    np.testing.assert_allclose(qo, y, atol=2e-6, rtol=0)
