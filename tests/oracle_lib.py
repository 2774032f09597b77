"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the compiled
reference harness (oracle/_ref/libref.so), plus seeded input builders.

Test infrastructure only: the product never imports this module.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")
REF_ENGINE_SO = os.path.join(ROOT, "oracle", "_ref", "libref_engine.so")

ORC_F32, ORC_F16, ORC_I8, ORC_FP8 = 0, 1, 2, 3
BS = 16  # reference BLOCK_SIZE (src/config.h:48)


class OrcPool(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("num_blocks", ctypes.c_int64),
        ("block_stride", ctypes.c_int64),
        ("scale_block_stride", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
    ]


_orc = None
_ref = None


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle not built: run `make -C oracle`")
        L = ctypes.CDLL(ORACLE_SO)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.orc_f16_encode_trunc.argtypes = [ctypes.c_float]
        L.orc_f16_encode_trunc.restype = ctypes.c_uint16
        L.orc_f16_encode_rne.argtypes = [ctypes.c_float]
        L.orc_f16_encode_rne.restype = ctypes.c_uint16
        L.orc_f16_decode.argtypes = [ctypes.c_uint16]
        L.orc_f16_decode.restype = ctypes.c_float
        L.orc_f16_encode_trunc_n.argtypes = [vp, vp, i64]
        L.orc_f16_decode_n.argtypes = [vp, vp, i64]
        L.orc_quant_i8.argtypes = [vp, i32, vp, vp]
        L.orc_fp8_encode.argtypes = [ctypes.c_float]
        L.orc_fp8_encode.restype = ctypes.c_uint8
        L.orc_fp8_decode.argtypes = [ctypes.c_uint8]
        L.orc_fp8_decode.restype = ctypes.c_float
        L.orc_fp8_encode_n.argtypes = [vp, vp, i64]
        L.orc_fp8_decode_n.argtypes = [vp, vp, i64]
        L.orc_quant_i8_rows.argtypes = [vp, i64, i32, vp, vp]
        L.orc_paged_attention.argtypes = [ctypes.POINTER(OrcPool), vp, vp, i32, i32, i32, vp]
        L.orc_decode_batch.argtypes = [ctypes.POINTER(OrcPool), vp, vp, i64, vp, vp, i32, i32,
                                       vp, i32]
        L.orc_prefill_batch.argtypes = [ctypes.POINTER(OrcPool), vp, vp, i64, vp, vp, i32, i32,
                                        vp, i32]
        L.orc_dense_f64.argtypes = [vp, vp, vp, i32, i32, ctypes.c_double, vp]
        L.orc_flash_attention.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]
        L.orc_partial.argtypes = [ctypes.POINTER(OrcPool), vp, i32, vp, i32, i32, i32, vp, vp, vp]
        L.orc_lse_merge.argtypes = [vp, vp, vp, i32, i32, vp]
        L.orc_fill_normal.argtypes = [ctypes.c_uint64, vp, i64, ctypes.c_double, ctypes.c_double]
        L.orc_fill_uniform_int.argtypes = [ctypes.c_uint64, vp, i64, i32, i32]
        L.orc_permutation.argtypes = [ctypes.c_uint64, vp, i32]
        L.orc_head_norm.argtypes = [vp, vp, ctypes.c_float, i64, i32]
        L.orc_rope.argtypes = [vp, i32, i32, i32, vp, vp, i32, i32]
        L.orc_rope_table.argtypes = [vp, vp, vp, vp, i32, i32, i32]
        _orc = L
    return _orc


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        L = ctypes.CDLL(REF_SO)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.ref_pool_create.argtypes = [i32, i32, i32, i32]
        L.ref_pool_create.restype = vp
        L.ref_pool_destroy.argtypes = [vp]
        L.ref_pool_write.argtypes = [vp, i32, vp, vp]
        L.ref_pool_read_raw.argtypes = [vp, i32, vp, vp]
        L.ref_fp8_encode_n.argtypes = [vp, vp, i64]
        L.ref_fp8_decode_n.argtypes = [vp, vp, i64]
        L.ref_decode.argtypes = [vp, i32, vp, vp, i64, vp, vp, i32, i32, i32, i32, vp]
        L.ref_prefill.argtypes = [vp, i32, vp, vp, i64, vp, vp, i32, i32, i32, i32, vp]
        _ref = L
    return _ref


# ---- seeded inputs ---------------------------------------------------------

def normal(seed, shape, mean=0.0, std=1.0):
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    orc().orc_fill_normal(seed, _p(out), n, mean, std)
    return out.reshape(shape)


def uniform_int(seed, n, lo, hi):
    out = np.empty(n, dtype=np.int32)
    orc().orc_fill_uniform_int(seed, _p(out), n, lo, hi)
    return out


def permutation(seed, n):
    out = np.empty(n, dtype=np.int32)
    orc().orc_permutation(seed, _p(out), n)
    return out


def f16_trunc(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty(x.shape, dtype=np.uint16)
    orc().orc_f16_encode_trunc_n(_p(x), _p(h), x.size)
    return h


def f16_decode(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    x = np.empty(h.shape, dtype=np.float32)
    orc().orc_f16_decode_n(_p(h), _p(x), h.size)
    return x


def fp8_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = np.empty(x.shape, dtype=np.uint8)
    orc().orc_fp8_encode_n(_p(x), _p(b), x.size)
    return b


def fp8_decode(b):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    x = np.empty(b.shape, dtype=np.float32)
    orc().orc_fp8_decode_n(_p(b), _p(x), b.size)
    return x


def quant_i8(x):
    """x [..., D] fp32 -> (int8 [..., D], fp16-bits scale [...])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.reshape(-1, D)
    q = np.empty(rows.shape, dtype=np.int8)
    s = np.empty(rows.shape[0], dtype=np.uint16)
    orc().orc_quant_i8_rows(_p(rows), rows.shape[0], D, _p(q), _p(s))
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


# ---- pools -------------------------------------------------------------------

class Pool:
    """Host pages in the reference per-layer slab layout [nb][BS][Hkv][D].
    kind F32: k/v float32; F16: uint16 bits; I8: int8 plus fp16-bit scales
    [nb][Hkv][BS]."""

    def __init__(self, kind, k, v, k_scale=None, v_scale=None, block_size=BS):
        self.kind, self.k, self.v = kind, np.ascontiguousarray(k), np.ascontiguousarray(v)
        self.k_scale = None if k_scale is None else np.ascontiguousarray(k_scale)
        self.v_scale = None if v_scale is None else np.ascontiguousarray(v_scale)
        self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim = k.shape
        assert block_size == self.block_size

    def orc_struct(self):
        nb, bs, hkv, d = self.k.shape
        s = OrcPool(self.kind, self.k.ctypes.data, self.v.ctypes.data,
                    None if self.k_scale is None else self.k_scale.ctypes.data,
                    None if self.v_scale is None else self.v_scale.ctypes.data,
                    nb, bs * hkv * d, hkv * bs, bs, hkv, d)
        return s

    def dequant(self):
        """fp32 K, V holding exactly the values the pool encodes."""
        if self.kind == ORC_F32:
            return self.k.astype(np.float32), self.v.astype(np.float32)
        if self.kind == ORC_F16:
            return f16_decode(self.k), f16_decode(self.v)
        if self.kind == ORC_FP8:
            return fp8_decode(self.k), fp8_decode(self.v)
        ks = f16_decode(self.k_scale).transpose(0, 2, 1)[..., None]  # [nb][BS][Hkv][1]
        vs = f16_decode(self.v_scale).transpose(0, 2, 1)[..., None]
        return (self.k.astype(np.float32) * ks).astype(np.float32), \
               (self.v.astype(np.float32) * vs).astype(np.float32)


def make_pool(kind, seed, num_blocks, num_kv_heads, head_dim, mean=0.0, std=1.0):
    shape = (num_blocks, BS, num_kv_heads, head_dim)
    k = normal(seed, shape, mean, std)
    v = normal(seed + 1, shape, mean, std)
    if kind == ORC_F32:
        return Pool(kind, k, v)
    if kind == ORC_F16:
        return Pool(kind, f16_trunc(k), f16_trunc(v))
    if kind == ORC_FP8:
        return Pool(kind, fp8_encode(k), fp8_encode(v))
    kq, ks = quant_i8(k)
    vq, vs = quant_i8(v)
    # scales [nb][BS][Hkv] -> [nb][Hkv][BS]
    return Pool(kind, kq, vq, np.ascontiguousarray(ks.transpose(0, 2, 1)),
                np.ascontiguousarray(vs.transpose(0, 2, 1)))


def decode(pool, q, tables, ctx, num_heads, table_lens=None, nthreads=8):
    q = np.ascontiguousarray(q, dtype=np.float32)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    ctx = np.ascontiguousarray(ctx, dtype=np.int32)
    tl = None if table_lens is None else np.ascontiguousarray(table_lens, dtype=np.int32)
    out = np.empty(q.shape, dtype=np.float32)
    s = pool.orc_struct()
    orc().orc_decode_batch(ctypes.byref(s), _p(q), _p(tables), tables.shape[1], _p(tl), _p(ctx),
                           q.shape[0], num_heads, _p(out), nthreads)
    return out


def prefill(pool, q, tables, q_start, prefix, num_heads, nthreads=8):
    q = np.ascontiguousarray(q, dtype=np.float32)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    q_start = np.ascontiguousarray(q_start, dtype=np.int32)
    prefix = np.ascontiguousarray(prefix, dtype=np.int32)
    out = np.empty(q.shape, dtype=np.float32)
    s = pool.orc_struct()
    orc().orc_prefill_batch(ctypes.byref(s), _p(q), _p(tables), tables.shape[1], _p(q_start),
                            _p(prefix), len(prefix), num_heads, _p(out), nthreads)
    return out


def single(pool, q, table, seq_len, num_heads):
    q = np.ascontiguousarray(q, dtype=np.float32)
    table = np.ascontiguousarray(table, dtype=np.int32)
    out = np.empty(q.shape, dtype=np.float32)
    s = pool.orc_struct()
    orc().orc_paged_attention(ctypes.byref(s), _p(q), _p(table), len(table), seq_len, num_heads,
                              _p(out))
    return out


# ---- compiled reference ------------------------------------------------------

class RefPool:
    """A reference KVCacheManager (FP32, FP16 or FP8_E4M3) filled through write_kv."""

    def __init__(self, k, v, fp16=False, fp8=False):
        nb, bs, hkv, d = k.shape
        assert bs == BS
        self.kv_dim = hkv * d
        self.num_kv_heads, self.head_dim = hkv, d
        self.h = ref().ref_pool_create(nb, 1, self.kv_dim, 2 if fp8 else 1 if fp16 else 0)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        ref().ref_pool_write(self.h, 0, _p(k), _p(v))
        self.shape = k.shape
        self.fp16, self.fp8 = fp16, fp8

    def raw(self):
        dt = np.uint8 if self.fp8 else np.uint16 if self.fp16 else np.float32
        k = np.empty(self.shape, dtype=dt)
        v = np.empty(self.shape, dtype=dt)
        ref().ref_pool_read_raw(self.h, 0, _p(k), _p(v))
        return k, v

    def decode(self, q, tables, ctx, num_heads, table_lens=None):
        q = np.ascontiguousarray(q, dtype=np.float32)
        tables = np.ascontiguousarray(tables, dtype=np.int32)
        ctx = np.ascontiguousarray(ctx, dtype=np.int32)
        tl = None if table_lens is None else np.ascontiguousarray(table_lens, dtype=np.int32)
        out = np.empty(q.shape, dtype=np.float32)
        ref().ref_decode(self.h, 0, _p(q), _p(tables), tables.shape[1], _p(tl), _p(ctx),
                         q.shape[0], num_heads, self.num_kv_heads, self.head_dim, _p(out))
        return out

    def prefill(self, q, tables, q_start, prefix, num_heads):
        q = np.ascontiguousarray(q, dtype=np.float32)
        tables = np.ascontiguousarray(tables, dtype=np.int32)
        q_start = np.ascontiguousarray(q_start, dtype=np.int32)
        prefix = np.ascontiguousarray(prefix, dtype=np.int32)
        out = np.empty(q.shape, dtype=np.float32)
        ref().ref_prefill(self.h, 0, _p(q), _p(tables), tables.shape[1], _p(q_start),
                          _p(prefix), len(prefix), num_heads, self.num_kv_heads, self.head_dim,
                          _p(out))
        return out

    def __del__(self):
        try:
            ref().ref_pool_destroy(self.h)
        except Exception:
            pass


def flash(q, k, v, mask=None):
    """orc_flash_attention on q [B][H][q_len][D], k/v [B][H][kv_len][D] (fp32);
    returns (out [B][H][D], weights [B*H][kv_len])."""
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    B, H, ql, D = q.shape
    kv = k.shape[2]
    out = np.zeros((B, H, D), np.float32)
    w = np.zeros((B * H, kv), np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, np.float32)
    orc().orc_flash_attention(_p(q), _p(k), _p(v), _p(out), _p(w), B, H, D, ql, kv,
                              None if m is None else _p(m))
    return out, w


# ---- query / key preparation ------------------------------------------------

ROPE_INTERLEAVED, ROPE_HALF = 0, 1


def head_norm(x, w, eps):
    """orc_head_norm on x [..., head_dim] (returns a new array)."""
    y = np.array(x, np.float32, copy=True, order="C")
    w = np.ascontiguousarray(w, np.float32)
    D = y.shape[-1]
    orc().orc_head_norm(_p(y), _p(w), ctypes.c_float(eps), y.size // D, D)
    return y


def rope(x, positions, inv_freq, style):
    """orc_rope on x [tokens][heads][head_dim] (returns a new array)."""
    y = np.array(x, np.float32, copy=True, order="C")
    T, H, D = y.shape
    pos = np.ascontiguousarray(positions, np.int32)
    f = np.ascontiguousarray(inv_freq, np.float32)
    orc().orc_rope(_p(y), T, H, D, _p(pos), _p(f), len(f), style)
    return y


def rope_table(q, k, cs, sn, head_dim):
    """orc_rope_table on q, k [batch][total_dim] (returns new arrays)."""
    q = np.array(q, np.float32, copy=True, order="C")
    k = np.array(k, np.float32, copy=True, order="C")
    cs = np.ascontiguousarray(cs, np.float32)
    sn = np.ascontiguousarray(sn, np.float32)
    B, total = q.shape
    orc().orc_rope_table(_p(q), _p(k), _p(cs), _p(sn), total, head_dim, B)
    return q, k


def inv_freq_table(head_dim, base=1000000.0):
    """The engine's default table: 1 / base^(2i / head_dim) in fp32
    (src/model.cpp:582-588, ROPE_BASE src/config.h:43)."""
    i = np.arange(head_dim // 2, dtype=np.float32)
    return (1.0 / np.power(np.float32(base), (np.float32(2.0) * i) / np.float32(head_dim))).astype(np.float32)


_ref_engine = None


def ref_engine_available():
    return os.path.exists(REF_ENGINE_SO)


def ref_engine():
    global _ref_engine
    if _ref_engine is None:
        L = ctypes.CDLL(REF_ENGINE_SO)
        vp, i32 = ctypes.c_void_p, ctypes.c_int32
        L.ref_rope_single.argtypes = [vp, i32, i32, i32, vp, i32]
        L.ref_rms_norm.argtypes = [vp, vp, vp, i32, ctypes.c_float]
        _ref_engine = L
    return _ref_engine
