"""GPU parity of the query/key preparation kernels against the oracle.

- vcpp_qk_norm_rope / vcpp_rope / vcpp_head_norm: the per-head RMS norm
  (src/paged_engine.cpp:14-20 per head) and RoPE at per-token positions
  (src/paged_engine.cpp:47-62; interleaved and half-split pairings).
  Tolerance |gpu - oracle| <= 1e-5 + 1e-5 |oracle|: the device sincosf and the
  lane-tree sum of squares differ from glibc's cosf/sinf and the sequential sum
  by a few fp32 ulps; every other operation is the same fp32 statement
  (contraction off).
- apply_rope_cuda (cuda/attention_kernels.cuh:249-287) is bit-exact: the same
  fp32 products and sums on the same cos/sin values.
- head_norm_cuda: the norm above through the v1 signature.
- config 3 size (16384 tokens x 64 q / 8 kv heads x 80): sampled tokens
  against the oracle, and the pair-length invariant on every row.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import dev

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-5


def close(got, want):
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def run_fused(q, k, pos, f, qw, kw, eps, style):
    qd = dev(q)
    kd = None if k is None else dev(k)
    pyvcpp.qk_norm_rope(qd, kd, None if pos is None else dev(np.asarray(pos, np.int32)),
                        None if f is None else dev(f), None if qw is None else dev(qw),
                        None if kw is None else dev(kw), eps, style)
    torch.cuda.synchronize()
    return qd.cpu().numpy(), None if kd is None else kd.cpu().numpy()


def want_fused(x, w, eps, pos, f, style):
    y = x
    if w is not None:
        y = O.head_norm(y, w, eps)
    if pos is not None:
        y = O.rope(y, pos, f, style)
    return y


@pytest.mark.parametrize("D", [64, 80, 128, 256])
@pytest.mark.parametrize("style", [pyvcpp.ROPE_INTERLEAVED, pyvcpp.ROPE_HALF])
@pytest.mark.parametrize("norm,rot", [(True, True), (False, True), (True, False)])
def test_fused_matches_oracle(D, style, norm, rot):
    T, H, HKV = 37, 8, 2
    q = O.normal(100 + D, (T, H, D), std=2.0)
    k = O.normal(200 + D, (T, HKV, D), std=2.0)
    pos = O.uniform_int(300 + D, T, 0, 40000) if rot else None
    pos = None if pos is None else np.asarray(pos, np.int32)
    if rot:
        pos[:3] = [0, 1, 131071]
    f = O.inv_freq_table(D) if rot else None
    qw = O.normal(400 + D, (D,), mean=1.0, std=0.2) if norm else None
    kw = O.normal(500 + D, (D,), mean=1.0, std=0.2) if norm else None
    eps = 1e-6
    gq, gk = run_fused(q, k, pos, f, qw, kw, eps, style)
    close(gq, want_fused(q, qw, eps, pos, f, style))
    close(gk, want_fused(k, kw, eps, pos, f, style))


def test_q_only_and_short_table():
    T, H, D = 9, 4, 80
    q = O.normal(7, (T, H, D))
    pos = np.arange(T, dtype=np.int32) * 1000
    f = O.inv_freq_table(D)[:5].copy()  # min(i, size - 1) clamp
    gq, _ = run_fused(q, None, pos, f, None, None, 0.0, pyvcpp.ROPE_INTERLEAVED)
    close(gq, O.rope(q, pos, f, O.ROPE_INTERLEAVED))


def test_rope_and_head_norm_entry_points():
    T, H, D = 21, 6, 80
    x = O.normal(8, (T, H, D), std=3.0)
    pos = np.asarray(O.uniform_int(9, T, 0, 5000), np.int32)
    f = O.inv_freq_table(D)
    xd = dev(x)
    pyvcpp.rope(xd, dev(pos), dev(f), pyvcpp.ROPE_HALF)
    torch.cuda.synchronize()
    close(xd.cpu().numpy(), O.rope(x, pos, f, O.ROPE_HALF))
    w = O.normal(10, (D,), mean=1.0, std=0.1)
    xd = dev(x)
    pyvcpp.head_norm(xd, dev(w), 1e-5)
    torch.cuda.synchronize()
    close(xd.cpu().numpy(), O.head_norm(x, w, 1e-5))
    # v1 head_norm_cuda, [B][H][D]
    xd = dev(x)
    pyvcpp.head_norm_cuda(xd, dev(w), 1e-5)
    close(xd.cpu().numpy(), O.head_norm(x, w, 1e-5))


@pytest.mark.parametrize("total,hd,B", [(640, 80, 3), (100, 80, 2), (6, 4, 1), (512, 128, 5)])
def test_apply_rope_cuda_bit_exact(total, hd, B):
    q = O.normal(11 + total, (B, total))
    k = O.normal(12 + total, (B, total))
    theta = O.inv_freq_table(hd) * np.float32(777)
    cs = np.cos(theta).astype(np.float32)
    sn = np.sin(theta).astype(np.float32)
    qd, kd = dev(q), dev(k)
    pyvcpp.apply_rope_cuda(qd, kd, dev(cs), dev(sn), hd)
    wq, wk = O.rope_table(q, k, cs, sn, hd)
    np.testing.assert_array_equal(qd.cpu().numpy(), wq)
    np.testing.assert_array_equal(kd.cpu().numpy(), wk)


def test_config3_size_sampled_and_invariant():
    """16384 prefill tokens at positions 1024..3071 (8 chunks of 2048 on a
    1024-token prefix), q_norm/k_norm then interleaved RoPE."""
    T, H, HKV, D = 16384, 64, 8, 80
    g = torch.Generator(device="cuda:0").manual_seed(3)
    q = torch.randn((T, H, D), generator=g, device="cuda:0")
    k = torch.randn((T, HKV, D), generator=g, device="cuda:0")
    pos = (torch.arange(T, dtype=torch.int32, device="cuda:0") % 2048) + 1024
    f = O.inv_freq_table(D)
    qw = O.normal(13, (D,), mean=1.0, std=0.1)
    kw = O.normal(14, (D,), mean=1.0, std=0.1)
    q0, k0 = q.clone(), k.clone()
    pyvcpp.qk_norm_rope(q, k, pos, dev(f), dev(qw), dev(kw), 1e-6, pyvcpp.ROPE_INTERLEAVED)
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(T, 64, replace=False)
    p = pos.cpu().numpy()[rows]
    close(q[rows].cpu().numpy(), want_fused(q0[rows].cpu().numpy(), qw, 1e-6, p, f, 0))
    close(k[rows].cpu().numpy(), want_fused(k0[rows].cpu().numpy(), kw, 1e-6, p, f, 0))
    # RoPE alone keeps each pair's length: every row of the full tensor
    x0 = torch.randn((T, H, D), generator=g, device="cuda:0")
    x = x0.clone()
    pyvcpp.rope(x, pos, dev(f), pyvcpp.ROPE_INTERLEAVED)
    n0 = torch.hypot(x0[..., 0::2], x0[..., 1::2])
    n1 = torch.hypot(x[..., 0::2], x[..., 1::2])
    assert torch.allclose(n1, n0, rtol=1e-5, atol=1e-6)
