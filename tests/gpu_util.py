"""Moves oracle pools and tables to the device and runs the library on them."""
import numpy as np
import torch

import pyvcpp
from oracle_lib import ORC_F16, ORC_F32, ORC_I8

KIND_TO_VCPP = {ORC_F32: pyvcpp.KV_F32, ORC_F16: pyvcpp.KV_F16, ORC_I8: pyvcpp.KV_I8}


def dev(a, device="cuda:0"):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(device)


class DevPool:
    """Device copy of an oracle_lib.Pool plus its vcpp_kv_pages descriptor."""

    def __init__(self, pool, device="cuda:0"):
        self.k = dev(pool.k, device)
        self.v = dev(pool.v, device)
        self.ks = None if pool.k_scale is None else dev(pool.k_scale, device)
        self.vs = None if pool.v_scale is None else dev(pool.v_scale, device)
        nb, bs, hkv, d = pool.k.shape
        self.pages = pyvcpp.kv_pages(KIND_TO_VCPP[pool.kind], self.k, self.v, bs, hkv, d, nb,
                                     bs * hkv * d, self.ks, self.vs, hkv * bs)


def gpu_decode(dpool, q, tables, ctx, num_heads, table_lens=None, partition_size=0,
               max_context_len=None):
    qd = dev(np.asarray(q, dtype=np.float32))
    out = torch.full_like(qd, float("nan"))
    td = dev(np.asarray(tables, dtype=np.int32))
    cd = dev(np.asarray(ctx, dtype=np.int32))
    tl = None if table_lens is None else dev(np.asarray(table_lens, dtype=np.int32))
    mcl = int(np.max(ctx)) if max_context_len is None else max_context_len
    pyvcpp.paged_decode(dpool.pages, qd, out, td, cd, mcl, num_heads, table_lens=tl,
                        partition_size=partition_size)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def assert_close(got, want, atol, rtol, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), "%s: non-finite output" % what
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), "%s: %d/%d out of tolerance, max abs err %.3g at %s" % (
        what, int(bad.sum()), bad.size, err.max(), np.unravel_index(err.argmax(), err.shape))
