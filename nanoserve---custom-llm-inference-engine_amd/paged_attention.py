"""Paged attention on MI355X: the reference's kernel surface over the gfx950 HIP library.

``paged_attention_hip`` takes the arguments of the reference's
``paged_attention_triton`` (nanoserve/kernels/paged_attention_triton.py:134-170) and
``paged_attention_torch`` (nanoserve/kernels/paged_attention_torch.py:31-100) in the same order
with the same meaning, and returns a tensor shaped and typed like ``query``. The computation runs in
``libns_paged_attention.so`` (include/ns_paged_attention.h); there is no other path: a missing
library raises.

Differences from the reference's launcher, all on the host side:
  * the per-query sequence index and KV position (paged_attention_triton.py:109-131) are found by
    the kernel itself from ``query_start_loc``, so no index tensors are built;
  * the grid's KV split needs the batch's longest sequence: ``max_seq_len`` (keyword) or, when
    omitted, ``int(seq_lens.max())`` -- one device-to-host read, as the reference's
    ``seq_lens.tolist()`` (paged_attention_triton.py:120, paged_attention_torch.py:51).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libns_paged_attention.so")

ABI_VERSION = 2
NS_PA_DTYPE_F32 = 0
NS_PA_DTYPE_BF16 = 1
NS_PA_DTYPE_F16 = 2
STATUS_BAD_BLOCK = 1
STATUS_SEQ_TOO_LONG = 2

EXPORTS = ("ns_pa_abi_version", "ns_pa_last_error", "ns_paged_attention_workspace_bytes",
           "ns_paged_attention")


class PagedAttentionError(RuntimeError):
    """An argument the library refused (the message is the library's)."""


class NsPagedAttnArgs(ctypes.Structure):
    """ns_paged_attn_args of include/ns_paged_attention.h, field for field."""

    _fields_ = [
        ("query", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("query_start_loc", ctypes.c_void_p),
        ("query_lens", ctypes.c_void_p),
        ("status", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("counters", ctypes.c_void_p),
        ("stride_q_token", ctypes.c_int64),
        ("stride_q_head", ctypes.c_int64),
        ("stride_k_block", ctypes.c_int64),
        ("stride_k_token", ctypes.c_int64),
        ("stride_k_head", ctypes.c_int64),
        ("stride_v_block", ctypes.c_int64),
        ("stride_v_token", ctypes.c_int64),
        ("stride_v_head", ctypes.c_int64),
        ("stride_o_token", ctypes.c_int64),
        ("stride_o_head", ctypes.c_int64),
        ("stride_bt_seq", ctypes.c_int64),
        ("total_q", ctypes.c_int32),
        ("num_seqs", ctypes.c_int32),
        ("num_heads_q", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
    ]


_LIB: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library (raises when it is not built: there is no fallback)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise PagedAttentionError(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    lib.ns_pa_abi_version.restype = ctypes.c_int
    lib.ns_pa_abi_version.argtypes = []
    lib.ns_pa_last_error.restype = ctypes.c_char_p
    lib.ns_pa_last_error.argtypes = []
    lib.ns_paged_attention_workspace_bytes.restype = ctypes.c_int
    lib.ns_paged_attention_workspace_bytes.argtypes = [ctypes.c_int32] * 5 + [ctypes.POINTER(ctypes.c_uint64)]
    lib.ns_paged_attention.restype = ctypes.c_int
    lib.ns_paged_attention.argtypes = [ctypes.POINTER(NsPagedAttnArgs), ctypes.c_void_p]
    if lib.ns_pa_abi_version() != ABI_VERSION:
        raise PagedAttentionError(f"ABI {lib.ns_pa_abi_version()} in {path}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def _check(rc: int) -> None:
    if rc != 0:
        raise PagedAttentionError(load().ns_pa_last_error().decode())


def workspace_bytes(total_q: int, num_heads_q: int, num_kv_heads: int, head_dim: int, max_seq_len: int) -> int:
    out = ctypes.c_uint64(0)
    _check(load().ns_paged_attention_workspace_bytes(total_q, num_heads_q, num_kv_heads, head_dim, max_seq_len,
                                                    ctypes.byref(out)))
    return int(out.value)


_COUNTERS = {}


def counters_for(device, n: int, stream=None):
    """A zero-filled int32 buffer of at least ``n`` arrival counters kept per device and stream
    (calls on one stream run one after another; calls on two streams may overlap, so they never
    share counters).  Every call leaves its counters at zero whatever its shape, so the buffer
    stays valid for all calls of its stream; it only grows, zero-filled on ``stream``."""
    import torch

    dev = torch.device(device)
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    key = (dev.index or 0, int(s.cuda_stream))
    buf = _COUNTERS.get(key)
    if buf is None or buf.numel() < n:
        with torch.cuda.stream(s):
            buf = torch.zeros(max(n, 1 << 16), dtype=torch.int32, device=dev)
        _COUNTERS[key] = buf
    return buf


def _dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: NS_PA_DTYPE_F32, torch.bfloat16: NS_PA_DTYPE_BF16, torch.float16: NS_PA_DTYPE_F16}
    if dtype not in codes:
        raise PagedAttentionError(f"unsupported dtype {dtype} (float32, bfloat16, float16)")
    return codes[dtype]


def _i32(t, device):
    import torch

    return t.to(device=device, dtype=torch.int32).contiguous()


def paged_attention_hip(query, k_cache, v_cache, block_tables, seq_lens, query_start_loc, query_lens,
                        scale: float, block_size: int, *, max_seq_len: Optional[int] = None,
                        out=None, workspace=None, counters=None, status=None, stream=None):
    """Attention of every query token over its sequence's paged KV (the reference's
    ``paged_attention_triton``; same arguments, same result up to float32 rounding order).

    query (total_q, Hq, D); k_cache/v_cache (num_blocks, block_size, Hkv, D) of query's dtype;
    block_tables int (num_seqs, max_blocks_per_seq); seq_lens, query_lens int (num_seqs);
    query_start_loc int (num_seqs + 1). ``status``, if given, is an int32 device tensor of one
    element that the kernel ORs STATUS_* bits into (a block id outside the cache, a sequence longer
    than ``max_seq_len``): a caller that wants the check reads it after the call. ``workspace``
    (uint8, any contents) and ``counters`` (int32, zero-filled once; every call leaves it so) are
    allocated per call, resp. taken from this module's per-device, per-stream buffer, when not
    given.  ``stream``: a ``torch.cuda.Stream`` or a raw HIP stream handle, default the current
    stream; the call's own temporaries are made on it, so nothing orders them against another.
    """
    import torch

    lib = load()
    dev = query.device
    if dev.type != "cuda":
        raise PagedAttentionError("paged_attention_hip needs device tensors")
    if stream is None:
        s = torch.cuda.current_stream(dev)
    elif isinstance(stream, torch.cuda.Stream):
        s = stream
    else:
        s = torch.cuda.ExternalStream(int(stream), device=dev)
    with torch.cuda.stream(s):
        return _paged_attention_on(lib, s, query, k_cache, v_cache, block_tables, seq_lens, query_start_loc,
                                   query_lens, scale, block_size, max_seq_len, out, workspace, counters, status)


def _paged_attention_on(lib, s, query, k_cache, v_cache, block_tables, seq_lens, query_start_loc, query_lens,
                        scale, block_size, max_seq_len, out, workspace, counters, status):
    """paged_attention_hip with ``s`` the current stream: every temporary below is made on it."""
    import torch

    dev = query.device
    total_q, hq, d = query.shape
    nb, bs, hkv, dk = k_cache.shape
    if v_cache.shape != k_cache.shape or dk != d:
        raise PagedAttentionError(f"cache shapes {tuple(k_cache.shape)}, {tuple(v_cache.shape)} do not match "
                                  f"the query's head_dim {d}")
    if k_cache.dtype != query.dtype or v_cache.dtype != query.dtype:
        raise PagedAttentionError("query and caches must share one dtype")
    if bs != block_size:
        raise PagedAttentionError(f"block_size {block_size} != the cache's {bs}")
    if total_q == 0:  # nothing to attend (an empty tensor's strides are arbitrary)
        return torch.empty_like(query) if out is None else out
    for name, t in (("query", query), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.stride(-1) != 1:
            raise PagedAttentionError(f"{name} must have a unit head_dim stride")
    bt = _i32(block_tables, dev)
    sl = _i32(seq_lens, dev)
    qsl = _i32(query_start_loc, dev)
    ql = _i32(query_lens, dev)
    num_seqs = bt.shape[0]
    if sl.numel() != num_seqs or ql.numel() != num_seqs or qsl.numel() != num_seqs + 1:
        raise PagedAttentionError("seq_lens/query_lens need num_seqs entries and query_start_loc num_seqs + 1")
    if max_seq_len is None:
        max_seq_len = int(sl.max().item()) if num_seqs else 0
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or out.device != dev:
        raise PagedAttentionError("out must match query's shape, dtype and device")
    elif out.stride(-1) != 1:
        raise PagedAttentionError("out must have a unit head_dim stride")
    need = workspace_bytes(total_q, hq, hkv, d, max_seq_len)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif need and workspace.numel() * workspace.element_size() < need:
        raise PagedAttentionError(f"workspace of {need} bytes needed")
    if need and counters is None:
        counters = counters_for(dev, total_q * hkv, s)
    elif need and (counters.dtype != torch.int32 or counters.device != dev or counters.numel() < total_q * hkv):
        raise PagedAttentionError(f"counters must be an int32 device tensor of at least {total_q * hkv} entries")
    if status is not None and (status.dtype != torch.int32 or status.device != dev or status.numel() < 1):
        raise PagedAttentionError("status must be an int32 device tensor")
    a = NsPagedAttnArgs(
        query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), bt.data_ptr(), sl.data_ptr(),
        qsl.data_ptr(), ql.data_ptr(), status.data_ptr() if status is not None else None,
        workspace.data_ptr() if need else None, need, counters.data_ptr() if need else None,
        query.stride(0), query.stride(1), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2), out.stride(0), out.stride(1),
        bt.stride(0) if bt.dim() == 2 else 0,
        total_q, num_seqs, hq, hkv, d, bs, nb, bt.shape[1] if bt.dim() == 2 else 0, max_seq_len,
        _dtype_code(query.dtype), float(scale))
    _check(lib.ns_paged_attention(ctypes.byref(a), ctypes.c_void_p(int(s.cuda_stream))))
    return out


# the reference's name, so that nanoserve/model/attention.py:21 can import this module unchanged
paged_attention_triton = paged_attention_hip
