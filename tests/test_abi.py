"""C-ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects bad arguments with a status code and a
message (argument validation runs before any HIP call)."""
import ctypes
import glob
import os
import re

import pytest

import pyvcpp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(", text, re.M):
            name = m.group(1)
            if name not in ("if", "while", "sizeof", "defined"):
                names.add(name)
    return names


def test_library_loads_and_exports_every_declared_symbol():
    L = pyvcpp.lib()
    names = declared_functions()
    assert "vcpp_paged_decode" in names and "paged_attention_cuda" in names
    for n in sorted(names):
        assert hasattr(L, n), "missing export %s" % n
    assert set(pyvcpp.EXPORTS) <= names


def test_version_and_error_string():
    assert b"gfx950" in pyvcpp.lib().vcpp_version()
    assert isinstance(pyvcpp.last_error(), str)


class FakeTensor:
    def __init__(self, addr, shape=(1,)):
        self._addr = addr
        self.shape = shape

    def data_ptr(self):
        return self._addr


def pages(dtype=pyvcpp.KV_F16, block_size=16, hkv=8, d=80, nb=10, stride=None, k=4096, v=8192):
    stride = block_size * hkv * d if stride is None else stride
    return pyvcpp.KVPages(dtype, block_size, hkv, d, nb, stride, 0, k, v, None, None)


def call(pg, num_seqs=1, num_heads=64, max_ctx=16, partition=0, q=4096, out=4096, ctx=4096,
         tables=4096, max_blocks=1, ws=None, ws_bytes=0):
    L = pyvcpp.lib()
    return L.vcpp_paged_decode(ctypes.byref(pg), q, out, tables, max_blocks, None, ctx, num_seqs,
                               max_ctx, num_heads, partition, ws, ws_bytes, None)


@pytest.mark.parametrize("kwargs,code,frag", [
    (dict(pg=pages(block_size=8)), pyvcpp.VCPP_E_UNSUPPORTED, "block_size"),
    (dict(pg=pages(d=72)), pyvcpp.VCPP_E_UNSUPPORTED, "head_dim"),
    (dict(pg=pages(dtype=7)), pyvcpp.VCPP_E_INVALID, "dtype"),
    (dict(pg=pages(), num_heads=60), pyvcpp.VCPP_E_INVALID, "num_heads"),
    (dict(pg=pages(), partition=24), pyvcpp.VCPP_E_INVALID, "partition"),
    (dict(pg=pages(k=4097)), pyvcpp.VCPP_E_INVALID, "aligned"),
    (dict(pg=pages(stride=16 * 8 * 80 - 8)), pyvcpp.VCPP_E_INVALID, "block_stride"),
    (dict(pg=pages(), q=None), pyvcpp.VCPP_E_INVALID, "NULL"),
    (dict(pg=pages(), max_ctx=100000, num_seqs=4), pyvcpp.VCPP_E_WORKSPACE, "workspace"),
    (dict(pg=pages(dtype=pyvcpp.KV_I8)), pyvcpp.VCPP_E_INVALID, "scale"),
])
def test_argument_errors(kwargs, code, frag):
    rc = call(**kwargs)
    assert rc == code
    assert frag in pyvcpp.last_error()


def test_empty_batch_is_a_no_op():
    assert call(pages(), num_seqs=0) == pyvcpp.VCPP_OK
    assert pyvcpp.last_error() == ""


def test_v1_rejects_block_size():
    L = pyvcpp.lib()
    ctx = (ctypes.c_int32 * 1)(16)
    L.paged_attention_cuda(4096, 4096, 4096, ctypes.addressof(ctx), 4096, 64, 8, 80, 8, 1)
    assert "block_size" in pyvcpp.last_error()


@pytest.mark.parametrize("heads,frag", [((64, 0), "num_kv_heads"), ((0, 8), "num_kv_heads"),
                                        ((60, 8), "num_kv_heads"), ((64, -8), "num_kv_heads")])
def test_v1_rejects_head_counts(heads, frag):
    """Head counts are checked before anything divides by them."""
    L = pyvcpp.lib()
    ctx = (ctypes.c_int32 * 1)(16)
    L.paged_attention_cuda(4096, 4096, 4096, ctypes.addressof(ctx), 4096, heads[0], heads[1], 80,
                           16, 1)
    assert frag in pyvcpp.last_error()


def test_v1_rejects_head_dim():
    L = pyvcpp.lib()
    ctx = (ctypes.c_int32 * 1)(16)
    L.paged_attention_cuda(4096, 4096, 4096, ctypes.addressof(ctx), 4096, 64, 8, 72, 16, 1)
    assert "head_dim 72" in pyvcpp.last_error()


def test_flash_rejects_empty_kv():
    """kv_len 0 would read an unset logit in the reference; here it records
    VCPP_E_INVALID before any HIP call."""
    L = pyvcpp.lib()
    dummy = ctypes.c_void_p(16)
    L.flash_attention_cuda(dummy, dummy, dummy, dummy, dummy, 1, 1, 80, 1, 0, None)
    assert "kv_len 0" in pyvcpp.last_error()
    L.flash_attention_cuda(None, dummy, dummy, dummy, dummy, 1, 1, 80, 1, 4, None)
    assert "NULL" in pyvcpp.last_error()


def test_qk_prep_argument_errors():
    """Shape, style and table checks of vcpp_qk_norm_rope / vcpp_rope /
    vcpp_head_norm run before any HIP call."""
    L = pyvcpp.lib()
    p = ctypes.c_void_p(4096)
    f = ctypes.c_float
    assert L.vcpp_qk_norm_rope(p, None, 4, 8, 0, 81, None, None, f(0), p, p, 40, 0, None) == \
        pyvcpp.VCPP_E_UNSUPPORTED
    assert "head_dim 81" in pyvcpp.last_error()
    assert L.vcpp_qk_norm_rope(p, None, 4, 8, 0, 512, None, None, f(0), p, p, 40, 0, None) == \
        pyvcpp.VCPP_E_UNSUPPORTED
    assert L.vcpp_qk_norm_rope(p, None, 4, 8, 0, 80, None, None, f(0), p, p, 40, 7, None) == \
        pyvcpp.VCPP_E_INVALID
    assert "style" in pyvcpp.last_error()
    assert L.vcpp_qk_norm_rope(p, None, 4, 8, 0, 80, None, None, f(0), p, None, 0, 0, None) == \
        pyvcpp.VCPP_E_INVALID
    assert "inv_freq" in pyvcpp.last_error()
    assert L.vcpp_qk_norm_rope(p, p, 4, 8, 0, 80, None, None, f(0), p, p, 40, 0, None) == \
        pyvcpp.VCPP_E_INVALID
    assert L.vcpp_qk_norm_rope(p, None, 4, 8, 0, 80, p, None, f(-1.0), None, None, 0, 0, None) == \
        pyvcpp.VCPP_E_INVALID
    assert "eps" in pyvcpp.last_error()
    assert L.vcpp_rope(p, 4, 8, 80, None, p, 40, 0, None) == pyvcpp.VCPP_E_INVALID
    assert L.vcpp_head_norm(p, None, f(1e-6), 4, 80, None) == pyvcpp.VCPP_E_INVALID
    # nothing to do: no launch, OK
    assert L.vcpp_qk_norm_rope(None, None, 0, 8, 0, 80, None, None, f(0), None, None, 0, 0, None) == \
        pyvcpp.VCPP_OK
    L.apply_rope_cuda(None, p, p, p, 160, 80, 2)
    assert "NULL" in pyvcpp.last_error()
    L.apply_rope_cuda(p, p, p, p, 160, 1, 2)
    assert "head_dim 1" in pyvcpp.last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No fallback path: without the built library the loader raises (and so
    does every op that needs it) instead of computing anything elsewhere."""
    monkeypatch.setattr(pyvcpp, "_lib", None)
    monkeypatch.setattr(pyvcpp, "LIB_PATH", str(tmp_path / "absent" / "libvcpp_attn.so"))
    with pytest.raises(RuntimeError, match="not built"):
        pyvcpp.lib()


@pytest.mark.parametrize("shape,hkv,heads,want", [
    # (chunks, max_chunk_len, max_prefix_len): one 512-token chunk on a 32 k
    # prefix: 8 tiles x 8 kv heads x 2 head groups = 128 workgroups -> 4 parts
    ((1, 512, 32768), 8, 64, 4 * 512 * 64 * 80 * 4 + 4 * 512 * 64 * 8),
    ((8, 2048, 1024), 8, 64, 0),       # config 3: 4096 workgroups fill the GPU
    ((1, 512, 0), 8, 64, 0),           # keys too short to split (512 + 0 keys: one part)
    ((1, 16, 6000), 1, 8, 11 * 16 * 8 * 80 * 4 + 11 * 16 * 8 * 8),  # (6000 + 16) / 512 = 11 parts
    ((1, 64, 100000), 1, 8, 16 * 64 * 8 * 80 * 4 + 16 * 64 * 8 * 8),  # at most 16 parts
])
def test_prefill_split_workspace_size(shape, hkv, heads, want):
    """The split prefill's part count and workspace ([parts][rows][heads]
    fp32 rows of head_dim, 256-byte aligned, then (max, sum) pairs) for a
    256-CU device (the count the library assumes without a device)."""
    L = pyvcpp.lib()
    pg = pages(hkv=hkv)
    assert L.vcpp_prefill_workspace_size(ctypes.byref(pg), *shape, heads) == want


def test_prefill_split_requires_workspace():
    L = pyvcpp.lib()
    pg = pages()
    rc = L.vcpp_paged_prefill_split(ctypes.byref(pg), 4096, 4096, 4096, 2048, 4096, 4096, 1, 512, 32768, 64,
                                    None, 0, None)
    assert rc == pyvcpp.VCPP_E_WORKSPACE
    assert "workspace" in pyvcpp.last_error()
