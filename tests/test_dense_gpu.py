"""GPU parity of flash_attention_cuda (the reference's contiguous-KV slot,
cuda/attention.cu:58-124) against the CPU restatement orc_flash_attention on
identical seeded inputs.  fp32 throughout: atol 1e-4, rtol 1e-4."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import pyvcpp
from gpu_util import assert_close, dev

pytestmark = pytest.mark.gpu


def run_gpu(q, k, v, mask=None):
    B, H, ql, D = q.shape
    kv = k.shape[2]
    qd, kd, vd = dev(q), dev(k), dev(v)
    out = torch.full((B, H, D), float("nan"), device="cuda:0")
    w = torch.full((B * H, kv), float("nan"), device="cuda:0")
    md = None if mask is None else dev(mask.astype(np.float32))
    pyvcpp.lib().flash_attention_cuda(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                      w.data_ptr(), B, H, D, ql, kv,
                                      None if md is None else md.data_ptr())
    torch.cuda.synchronize()
    assert pyvcpp.last_error() == ""
    return out.cpu().numpy(), w.cpu().numpy()


# Shapes cover the LDS-DMA one-pass kernel (head_dim 64/80/96/128: fewer
# chunks than waves, ragged last chunks, exactly one 4096-key logit segment,
# one key past it, three segments) and the plain kernel at another head dim.
@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 80), (2, 8, 3, 300, 80), (3, 4, 1, 1000, 128),
                                   (1, 2, 2, 17, 64), (1, 1, 1, 5000, 96), (1, 1, 1, 48, 64),
                                   (1, 4, 1, 33, 128), (2, 3, 1, 4096, 96), (1, 2, 1, 4096, 80),
                                   (1, 2, 1, 4097, 80), (1, 2, 1, 9001, 64), (1, 1, 1, 12288, 128),
                                   (2, 2, 1, 777, 48)])
def test_flash_matches_oracle(cuda, shape):
    B, H, ql, kv, D = shape
    q = O.normal(1000 + kv, (B, H, ql, D))
    k = O.normal(2000 + kv, (B, H, kv, D))
    v = O.normal(3000 + kv, (B, H, kv, D))
    want, want_w = O.flash(q, k, v)
    got, got_w = run_gpu(q, k, v)
    assert_close(got, want, 1e-4, 1e-4, what="flash out %s" % (shape,))
    assert_close(got_w, want_w, 1e-5, 1e-4, what="flash weights %s" % (shape,))


def test_flash_mask(cuda):
    B, H, ql, kv, D = 2, 3, 1, 200, 80
    q = O.normal(11, (B, H, ql, D))
    k = O.normal(12, (B, H, kv, D))
    v = O.normal(13, (B, H, kv, D))
    mask = np.where(O.normal(14, (kv,)) > 0.3, 0.0, -1.0).astype(np.float32)
    want, want_w = O.flash(q, k, v, mask)
    got, got_w = run_gpu(q, k, v, mask)
    assert_close(got, want, 1e-4, 1e-4, what="flash masked out")
    assert_close(got_w, want_w, 1e-5, 1e-4, what="flash masked weights")
    assert np.all(got_w[:, mask < 0] == 0.0)


@pytest.mark.parametrize("shape", [(1, 2, 1, 33, 64), (2, 3, 1, 200, 80), (1, 2, 1, 4100, 96),
                                   (1, 1, 1, 8200, 128), (1, 1, 1, 100, 48)])
def test_flash_mask_shapes(cuda, shape):
    """Masks through the one-pass kernel's DMA ring (and the plain kernel at
    head_dim 48): masked keys get probability 0 and leave the output."""
    B, H, ql, kv, D = shape
    q = O.normal(21 + kv, (B, H, ql, D))
    k = O.normal(22 + kv, (B, H, kv, D))
    v = O.normal(23 + kv, (B, H, kv, D))
    mask = np.where(O.normal(24 + kv, (kv,)) > 0.0, 0.0, -1.0).astype(np.float32)
    want, want_w = O.flash(q, k, v, mask)
    got, got_w = run_gpu(q, k, v, mask)
    assert_close(got, want, 1e-4, 1e-4, what="flash masked out %s" % (shape,))
    assert_close(got_w, want_w, 1e-5, 1e-4, what="flash masked weights %s" % (shape,))
    assert np.all(got_w[:, mask < 0] == 0.0)


def test_flash_all_masked(cuda):
    """Every key masked: the reference's -1e9 logits give uniform weights."""
    B, H, ql, kv, D = 1, 2, 1, 50, 80
    q = O.normal(31, (B, H, ql, D))
    k = O.normal(32, (B, H, kv, D))
    v = O.normal(33, (B, H, kv, D))
    mask = np.full((kv,), -1.0, dtype=np.float32)
    want, want_w = O.flash(q, k, v, mask)
    got, got_w = run_gpu(q, k, v, mask)
    assert_close(got, want, 1e-4, 1e-4, what="flash all masked out")
    assert_close(got_w, want_w, 1e-5, 1e-4, what="flash all masked weights")


_CHILD = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[2])
import pyvcpp
a = np.load(sys.argv[1] + "/in.npz")
outs = {}
for i in range(int(a["n"])):
    q, k, v = (torch.from_numpy(a["%s%d" % (x, i)]).to("cuda:0") for x in "qkv")
    m = a["m%d" % i]
    md = torch.from_numpy(m).to("cuda:0") if m.size else None
    B, H, ql, D = q.shape
    kv = k.shape[2]
    out = torch.full((B, H, D), float("nan"), device="cuda:0")
    w = torch.full((B * H, kv), float("nan"), device="cuda:0")
    pyvcpp.lib().flash_attention_cuda(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), w.data_ptr(),
                                      B, H, D, ql, kv, None if md is None else md.data_ptr())
    torch.cuda.synchronize()
    assert pyvcpp.last_error() == ""
    outs["o%d" % i] = out.cpu().numpy()
    outs["w%d" % i] = w.cpu().numpy()
np.savez(sys.argv[1] + "/out.npz", **outs)
"""


def test_flash_register_kernels(cuda, tmp_path):
    """The register-load kernels (dense_attention_vec_kernel at head_dim
    64 / 80 / 128, kept behind VCPP_DENSE_DMA=0, which the library reads once
    per process): one child process runs a few shapes with the switch set."""
    import os
    import subprocess
    import sys
    shapes = [(2, 3, 1, 300, 64, False), (1, 4, 2, 1000, 80, True), (1, 2, 1, 5000, 128, False)]
    arrays, wants = {"n": np.array(len(shapes))}, []
    for i, (B, H, ql, kv, D, masked) in enumerate(shapes):
        q = O.normal(41 + i, (B, H, ql, D))
        k = O.normal(51 + i, (B, H, kv, D))
        v = O.normal(61 + i, (B, H, kv, D))
        mask = np.where(O.normal(71 + i, (kv,)) > 0.0, 0.0, -1.0).astype(np.float32) if masked else None
        arrays.update({"q%d" % i: q.astype(np.float32), "k%d" % i: k.astype(np.float32),
                       "v%d" % i: v.astype(np.float32),
                       "m%d" % i: mask if masked else np.zeros((0,), np.float32)})
        wants.append(O.flash(q, k, v, mask))
    np.savez(tmp_path / "in.npz", **arrays)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, VCPP_DENSE_DMA="0")
    r = subprocess.run([sys.executable, "-c", _CHILD, str(tmp_path), os.path.join(root, "vllm-cpp_amd")],
                       env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    got = np.load(tmp_path / "out.npz")
    for i, (want, want_w) in enumerate(wants):
        assert_close(got["o%d" % i], want, 1e-4, 1e-4, what="flash register kernels out %s" % (shapes[i],))
        assert_close(got["w%d" % i], want_w, 1e-5, 1e-4, what="flash register kernels weights %s" % (shapes[i],))
