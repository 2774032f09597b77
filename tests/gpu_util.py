"""Moves oracle pools and tables to the device and runs the library on them."""
import numpy as np
import torch

import pyvcpp
from oracle_lib import ORC_F16, ORC_F32, ORC_FP8, ORC_I8

KIND_TO_VCPP = {ORC_F32: pyvcpp.KV_F32, ORC_F16: pyvcpp.KV_F16, ORC_I8: pyvcpp.KV_I8,
                ORC_FP8: pyvcpp.KV_FP8}


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


# (what, max-abs error, normwise relative error, atol, rtol) of every check this
# session; conftest prints them in the terminal summary.
PARITY_LOG = []


def assert_close(got, want, atol, rtol, what=""):
    """The parity bar, both halves outright: max |got - want| <= atol, and the
    normwise relative error ||got - want||_2 / ||want||_2 <= rtol (an
    elementwise relative bound is meaningless where outputs cross zero)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), "%s: non-finite output" % what
    err = np.abs(got - want)
    max_abs = float(err.max()) if err.size else 0.0
    norm = float(np.linalg.norm(want))
    rel = float(np.linalg.norm(err)) / norm if norm > 0 else float(np.linalg.norm(err))
    PARITY_LOG.append((what, max_abs, rel, atol, rtol))
    assert max_abs <= atol, "%s: max abs err %.3g > %.3g at %s (%d/%d elements above)" % (
        what, max_abs, atol, np.unravel_index(err.argmax(), err.shape), int((err > atol).sum()),
        err.size)
    assert rel <= rtol, "%s: normwise relative err %.3g > %.3g" % (what, rel, rtol)


def prefill_tables(seed, lens, num_blocks, bs=16):
    """Random disjoint block tables for sequences of `lens` tokens."""
    from oracle_lib import permutation
    nbs = [(n + bs - 1) // bs for n in lens]
    mb = max(max(nbs), 1)
    perm = permutation(seed, num_blocks)
    t = np.full((len(lens), mb), -1, dtype=np.int32)
    k = 0
    for i, n in enumerate(nbs):
        t[i, :n] = perm[k:k + n]
        k += n
    assert k <= num_blocks
    return t


def gpu_prefill(dpool, q16, tables, q_start, prefix, num_heads):
    """q16: uint16 fp16 bits [rows][H][D]."""
    qd = dev(q16)
    out = torch.full(q16.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    lens = np.diff(q_start)
    pyvcpp.paged_prefill(dpool.pages, qd, out, dev(np.asarray(tables, np.int32)),
                         dev(np.asarray(q_start, np.int32)), dev(np.asarray(prefix, np.int32)),
                         int(lens.max()) if len(lens) else 0, num_heads)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_prefill_rows(pool, q32, tables, q_start, prefix, num_heads, rows, nthreads=8):
    """Oracle for selected query rows only: each row is a single-token query
    over positions 0..prefix+i of its chunk (the engine's per-position
    semantics), evaluated with the batched decode oracle."""
    from oracle_lib import decode
    chunk_of = np.searchsorted(q_start, rows, side="right") - 1
    ctx = np.array([prefix[c] + (r - q_start[c]) + 1 for r, c in zip(rows, chunk_of)], np.int32)
    return decode(pool, q32[rows], tables[chunk_of], ctx, num_heads, nthreads=nthreads)


def gpu_prefill_split(dpool, q16, tables, q_start, prefix, num_heads, workspace=None):
    """vcpp_paged_prefill_split; returns (out, splits used > 1)."""
    qd = dev(q16)
    out = torch.full(q16.shape, float("nan"), dtype=torch.float32, device="cuda:0")
    lens = np.diff(q_start)
    mcl = int(lens.max()) if len(lens) else 0
    mpl = int(np.max(prefix)) if len(prefix) else 0
    need = pyvcpp.prefill_workspace_size(dpool.pages, len(lens), mcl, mpl, num_heads)
    pyvcpp.paged_prefill_split(dpool.pages, qd, out, dev(np.asarray(tables, np.int32)),
                               dev(np.asarray(q_start, np.int32)), dev(np.asarray(prefix, np.int32)),
                               mcl, mpl, num_heads, workspace=workspace)
    torch.cuda.synchronize()
    return out.cpu().numpy(), need > 0
