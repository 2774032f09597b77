"""ctypes binding of libvcpp_attn.so (include/vcpp_attention.h).

Tests and bench.py call the library only through this module, i.e. through
the C ABI.  Torch tensors are used as device-memory plumbing (data_ptr() and
the current HIP stream); nothing here computes attention.  Loading fails
loudly when the library has not been built -- there is no fallback path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# VCPP_ATTN_LIB selects another build of the library (e.g. a kernel variant).
LIB_PATH = os.environ.get("VCPP_ATTN_LIB") or os.path.join(HERE, "libvcpp_attn.so")

VCPP_OK = 0
VCPP_E_INVALID = -1
VCPP_E_UNSUPPORTED = -2
VCPP_E_WORKSPACE = -3
VCPP_E_HIP = -4

KV_F32 = 0
KV_F16 = 1
KV_I8 = 2
KV_FP8 = 3

# Every symbol include/vcpp_attention.h declares.
EXPORTS = [
    "vcpp_last_error",
    "vcpp_version",
    "vcpp_paged_decode",
    "vcpp_paged_decode_noalloc",
    "vcpp_decode_workspace_size",
    "vcpp_paged_prefill",
    "vcpp_write_kv",
    "vcpp_qk_norm_rope",
    "vcpp_rope",
    "vcpp_head_norm",
    "apply_rope_cuda",
    "head_norm_cuda",
    "paged_attention_cuda",
    "flash_attention_cuda",
    "vcpp_profile_enable",
    "vcpp_profile_read",
]

KERNEL_DECODE, KERNEL_MERGE, KERNEL_PREFILL, KERNEL_MIXED = 0, 1, 2, 3


class KVPages(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("num_blocks", ctypes.c_int64),
        ("block_stride", ctypes.c_int64),
        ("scale_block_stride", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
    ]


class VcppError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("vcpp error %d: %s" % (code, msg))
        self.code = code


_lib = None


def lib():
    """Loads libvcpp_attn.so once; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            "libvcpp_attn.so not built (%s); run __graft_entry__.build()" % LIB_PATH)
    _lib = open_library(LIB_PATH)
    return _lib


GATHER_LIB_PATH = os.path.join(HERE, "libvcpp_attn_gather.so")


def open_library(path):
    """Loads a build of the library at `path` with every entry point's
    argument types set (lib() loads the product build; tests also open the
    gather-index checker build, GATHER_LIB_PATH)."""
    if not os.path.exists(path):
        raise RuntimeError("%s not built; run __graft_entry__.build()" % path)
    L = ctypes.CDLL(path)
    L.vcpp_last_error.restype = ctypes.c_char_p
    L.vcpp_version.restype = ctypes.c_char_p
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    L.vcpp_paged_decode.argtypes = [ctypes.POINTER(KVPages), vp, vp, vp, i32, vp, vp, i32, i32,
                                    i32, i32, vp, sz, vp]
    L.vcpp_paged_decode.restype = ctypes.c_int
    L.vcpp_paged_decode_noalloc.argtypes = [ctypes.POINTER(KVPages), vp, vp, vp, i32, vp, vp, i32,
                                            i32, i32, i32, vp]
    L.vcpp_paged_decode_noalloc.restype = ctypes.c_int
    L.vcpp_decode_workspace_size.argtypes = [ctypes.POINTER(KVPages), i32, i32, i32, i32]
    L.vcpp_decode_workspace_size.restype = sz
    L.vcpp_paged_prefill.argtypes = [ctypes.POINTER(KVPages), vp, vp, vp, i32, vp, vp, i32, i32,
                                     i32, vp]
    L.vcpp_paged_prefill.restype = ctypes.c_int
    L.vcpp_paged_prefill_split.argtypes = [ctypes.POINTER(KVPages), vp, vp, vp, i32, vp, vp, i32, i32, i32,
                                           i32, vp, sz, vp]
    L.vcpp_paged_prefill_split.restype = ctypes.c_int
    L.vcpp_prefill_workspace_size.argtypes = [ctypes.POINTER(KVPages), i32, i32, i32, i32]
    L.vcpp_prefill_workspace_size.restype = sz
    L.vcpp_paged_mixed_step.argtypes = [ctypes.POINTER(KVPages), vp, vp, vp, i32, vp, vp, i32, i32,
                                        vp, vp, vp, i32, vp, vp, i32, i32, i32, vp, sz, vp]
    L.vcpp_paged_mixed_step.restype = ctypes.c_int
    L.vcpp_mixed_workspace_size.argtypes = [ctypes.POINTER(KVPages), i32, i32, i32, i32]
    L.vcpp_mixed_workspace_size.restype = sz
    L.vcpp_write_kv.argtypes = [ctypes.POINTER(KVPages), vp, vp, vp, i32, i32, vp]
    L.vcpp_write_kv.restype = ctypes.c_int
    L.vcpp_qk_norm_rope.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, ctypes.c_float, vp, vp,
                                    i32, i32, vp]
    L.vcpp_qk_norm_rope.restype = ctypes.c_int
    L.vcpp_rope.argtypes = [vp, i32, i32, i32, vp, vp, i32, i32, vp]
    L.vcpp_rope.restype = ctypes.c_int
    L.vcpp_head_norm.argtypes = [vp, vp, ctypes.c_float, i32, i32, vp]
    L.vcpp_head_norm.restype = ctypes.c_int
    L.apply_rope_cuda.argtypes = [vp, vp, vp, vp, i32, i32, i32]
    L.apply_rope_cuda.restype = None
    L.head_norm_cuda.argtypes = [vp, vp, ctypes.c_float, i32, i32, i32]
    L.head_norm_cuda.restype = None
    L.paged_attention_cuda.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]
    L.paged_attention_cuda.restype = None
    L.flash_attention_cuda.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]
    L.flash_attention_cuda.restype = None
    L.vcpp_profile_enable.argtypes = [ctypes.c_int]
    L.vcpp_profile_enable.restype = ctypes.c_int
    L.vcpp_profile_read.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_int64)]
    L.vcpp_profile_read.restype = ctypes.c_int
    if hasattr(L, "vcpp_debug_gather_dump"):
        L.vcpp_debug_gather_dump.argtypes = [vp, i64]
        L.vcpp_debug_gather_dump.restype = None
    return L


def last_error():
    return lib().vcpp_last_error().decode()


def _check(rc):
    if rc != VCPP_OK:
        raise VcppError(rc, last_error())


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def kv_pages(dtype, k, v, block_size, num_kv_heads, head_dim, num_blocks, block_stride,
             k_scale=None, v_scale=None, scale_block_stride=0):
    """Builds a vcpp_kv_pages descriptor from device tensors (kept alive by caller)."""
    return KVPages(dtype, block_size, num_kv_heads, head_dim, num_blocks, block_stride,
                   scale_block_stride, k.data_ptr(), v.data_ptr(),
                   None if k_scale is None else k_scale.data_ptr(),
                   None if v_scale is None else v_scale.data_ptr())


def decode_workspace_size(pages, num_seqs, num_heads, max_context_len, partition_size=0):
    return lib().vcpp_decode_workspace_size(ctypes.byref(pages), num_seqs, num_heads,
                                            max_context_len, partition_size)


def paged_decode(pages, q, out, block_tables, context_lens, max_context_len, num_heads,
                 table_lens=None, partition_size=0, workspace=None, stream=None):
    """vcpp_paged_decode on device tensors.  `workspace` is a uint8 device
    tensor of at least decode_workspace_size(...) bytes, reusable across calls
    on one stream (allocated here when None)."""
    num_seqs = q.shape[0]
    max_blocks = block_tables.shape[1] if block_tables is not None and block_tables.dim() == 2 else 0
    need = decode_workspace_size(pages, num_seqs, num_heads, max_context_len, partition_size)
    if workspace is None and need > 0:
        import torch
        workspace = torch.zeros(need, dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() if workspace is not None else 0
    rc = lib().vcpp_paged_decode(ctypes.byref(pages), _ptr(q), _ptr(out), _ptr(block_tables),
                                 max_blocks, _ptr(table_lens), _ptr(context_lens), num_seqs,
                                 max_context_len, num_heads, partition_size, _ptr(workspace),
                                 ws_bytes, _stream(stream))
    _check(rc)
    return out


def paged_decode_noalloc(pages, q, out, block_tables, context_lens, max_context_len, num_heads,
                         table_lens=None, partition_size=0, stream=None):
    """vcpp_paged_decode_noalloc: as paged_decode, with the library's static
    split-K scratch instead of a workspace (allocates nothing)."""
    num_seqs = q.shape[0]
    max_blocks = block_tables.shape[1] if block_tables is not None and block_tables.dim() == 2 else 0
    rc = lib().vcpp_paged_decode_noalloc(ctypes.byref(pages), _ptr(q), _ptr(out), _ptr(block_tables),
                                         max_blocks, _ptr(table_lens), _ptr(context_lens), num_seqs,
                                         max_context_len, num_heads, partition_size, _stream(stream))
    _check(rc)
    return out


def profile_enable(on=True):
    _check(lib().vcpp_profile_enable(1 if on else 0))


def profile_read(kernel_id):
    """(total_ms, launches) of one kernel since the last profile_enable()."""
    ms = ctypes.c_double()
    n = ctypes.c_int64()
    _check(lib().vcpp_profile_read(kernel_id, ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def paged_prefill(pages, q, out, block_tables, q_start, prefix_lens, max_chunk_len, num_heads,
                  stream=None):
    """vcpp_paged_prefill on device tensors (q fp16, out fp32)."""
    rc = lib().vcpp_paged_prefill(ctypes.byref(pages), _ptr(q), _ptr(out), _ptr(block_tables),
                                  block_tables.shape[1], _ptr(q_start), _ptr(prefix_lens),
                                  prefix_lens.shape[0], max_chunk_len, num_heads, _stream(stream))
    _check(rc)
    return out


def mixed_workspace_size(pages, num_seqs, num_heads, max_context_len, max_blocks_per_chunk):
    return lib().vcpp_mixed_workspace_size(ctypes.byref(pages), num_seqs, num_heads, max_context_len,
                                           max_blocks_per_chunk)


def paged_mixed_step(pages, dq, dout, d_tables, context_lens, max_context_len, pq, pout, p_tables,
                     q_start, prefix_lens, max_chunk_len, num_heads, d_table_lens=None,
                     workspace=None, stream=None):
    """vcpp_paged_mixed_step: a decode batch (dq fp32 [S][H][D]) and prefill
    chunks (pq fp16 [rows][H][D]) over the same pages in one step."""
    num_seqs = dq.shape[0] if dq is not None else 0
    num_chunks = prefix_lens.shape[0] if prefix_lens is not None else 0
    dmb = d_tables.shape[1] if d_tables is not None and d_tables.dim() == 2 else 0
    pmb = p_tables.shape[1] if p_tables is not None and p_tables.dim() == 2 else 0
    need = mixed_workspace_size(pages, num_seqs, num_heads, max_context_len, pmb)
    if workspace is None and need > 0:
        import torch
        workspace = torch.zeros(need, dtype=torch.uint8, device=dq.device)
    ws_bytes = workspace.numel() if workspace is not None else 0
    rc = lib().vcpp_paged_mixed_step(ctypes.byref(pages), _ptr(dq), _ptr(dout), _ptr(d_tables), dmb,
                                     _ptr(d_table_lens), _ptr(context_lens), num_seqs, max_context_len,
                                     _ptr(pq), _ptr(pout), _ptr(p_tables), pmb, _ptr(q_start),
                                     _ptr(prefix_lens), num_chunks, max_chunk_len, num_heads,
                                     _ptr(workspace), ws_bytes, _stream(stream))
    _check(rc)


def prefill_workspace_size(pages, num_chunks, max_chunk_len, max_prefix_len, num_heads):
    return lib().vcpp_prefill_workspace_size(ctypes.byref(pages), num_chunks, max_chunk_len, max_prefix_len,
                                             num_heads)


def paged_prefill_split(pages, q, out, block_tables, q_start, prefix_lens, max_chunk_len, max_prefix_len,
                        num_heads, workspace=None, stream=None):
    """vcpp_paged_prefill_split on device tensors (q fp16, out fp32)."""
    nc = prefix_lens.shape[0]
    need = prefill_workspace_size(pages, nc, max_chunk_len, max_prefix_len, num_heads)
    if workspace is None and need > 0:
        import torch
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() if workspace is not None else 0
    rc = lib().vcpp_paged_prefill_split(ctypes.byref(pages), _ptr(q), _ptr(out), _ptr(block_tables),
                                        block_tables.shape[1], _ptr(q_start), _ptr(prefix_lens), nc,
                                        max_chunk_len, max_prefix_len, num_heads, _ptr(workspace), ws_bytes,
                                        _stream(stream))
    _check(rc)
    return out


def write_kv(pages, k, v, slots, fp16_round_nearest=False, stream=None):
    """vcpp_write_kv: k, v fp32 [n][Hkv][D] and slots int64 [n] device tensors."""
    rc = lib().vcpp_write_kv(ctypes.byref(pages), _ptr(k), _ptr(v), _ptr(slots), k.shape[0],
                             1 if fp16_round_nearest else 0, _stream(stream))
    _check(rc)


ROPE_INTERLEAVED, ROPE_HALF = 0, 1


def qk_norm_rope(q, k=None, positions=None, inv_freq=None, q_norm_weight=None, k_norm_weight=None,
                 eps=1e-6, style=ROPE_INTERLEAVED, stream=None):
    """vcpp_qk_norm_rope in place on q [T][H][D] and k [T][Hkv][D] (fp32 device tensors)."""
    T, H, D = q.shape
    Hkv = k.shape[1] if k is not None else 0
    nf = inv_freq.numel() if inv_freq is not None else 0
    rc = lib().vcpp_qk_norm_rope(_ptr(q), _ptr(k), T, H, Hkv, D, _ptr(q_norm_weight),
                                 _ptr(k_norm_weight), ctypes.c_float(eps), _ptr(positions),
                                 _ptr(inv_freq), nf, style, _stream(stream))
    _check(rc)


def rope(x, positions, inv_freq, style=ROPE_INTERLEAVED, stream=None):
    """vcpp_rope in place on x [T][H][D]."""
    T, H, D = x.shape
    _check(lib().vcpp_rope(_ptr(x), T, H, D, _ptr(positions), _ptr(inv_freq), inv_freq.numel(),
                           style, _stream(stream)))


def head_norm(x, weight, eps, stream=None):
    """vcpp_head_norm in place on x [..., D]."""
    D = x.shape[-1]
    _check(lib().vcpp_head_norm(_ptr(x), _ptr(weight), ctypes.c_float(eps), x.numel() // D, D,
                                _stream(stream)))


def apply_rope_cuda(q, k, cos, sin, head_dim):
    """v1 apply_rope_cuda on q, k [B][total_dim]; raises on a recorded error."""
    B, total = q.shape
    lib().apply_rope_cuda(_ptr(q), _ptr(k), _ptr(cos), _ptr(sin), total, head_dim, B)
    err = last_error()
    if err:
        raise VcppError(VCPP_E_INVALID, err)


def head_norm_cuda(x, weight, eps):
    """v1 head_norm_cuda on x [B][H][D]; raises on a recorded error."""
    B, H, D = x.shape
    lib().head_norm_cuda(_ptr(x), _ptr(weight), ctypes.c_float(eps), H, D, B)
    err = last_error()
    if err:
        raise VcppError(VCPP_E_INVALID, err)
