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


# Shapes cover both kernel families: the LDS-DMA one-pass kernel (no mask,
# kv_len <= 4096, head_dim 64/80/96/128: fewer chunks than waves, ragged last
# chunks, exactly 4096 keys) and the register-load kernels past 4096 keys or at
# other head dims.
@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 80), (2, 8, 3, 300, 80), (3, 4, 1, 1000, 128),
                                   (1, 2, 2, 17, 64), (1, 1, 1, 5000, 96), (1, 1, 1, 48, 64),
                                   (1, 4, 1, 33, 128), (2, 3, 1, 4096, 96), (1, 2, 1, 4096, 80),
                                   (1, 2, 1, 4097, 80), (2, 2, 1, 777, 48)])
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
