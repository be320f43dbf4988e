"""Paged attention on MI355X: the reference's kernel surface over the gfx950 HIP library.

``paged_attention_hip`` takes the arguments of the reference's
``paged_attention_triton`` (nanoserve/kernels/paged_attention_triton.py:134-170) and
``paged_attention_torch`` (nanoserve/kernels/paged_attention_torch.py:31-100) in the same order
with the same meaning, and returns a tensor shaped and typed like ``query``. The computation runs in
``libns_paged_attention.so`` (include/ns_paged_attention.h); there is no other path: a missing
library raises.

Differences from the reference's launcher, all on the host side:
  * decode batches (every ``query_lens`` entry 1, declared by ``max_query_len=1``): the
    per-query sequence index and KV position (paged_attention_triton.py:109-131) are found by
    the kernel itself from ``query_start_loc``, so no index tensors are built, and with
    ``max_seq_len`` given the call reads nothing on the host;
  * otherwise the batch layout (``seq_lens``, ``query_start_loc``, ``query_lens``) is read on the
    host once, as the reference's launcher reads ``seq_lens.tolist()`` and ``query_lens.tolist()``
    (paged_attention_triton.py:120-121, paged_attention_torch.py:51): sequences of at least
    ``PREFILL_MIN_QUERY`` query tokens (bfloat16 and float16) are cut into query tiles of
    ``64 // G`` tokens for the MFMA prefill kernel, which reads each key and value row once per
    tile; the other query tokens go to the per-token kernel.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libns_paged_attention.so")

ABI_VERSION = 3
NS_PA_DTYPE_F32 = 0
NS_PA_DTYPE_BF16 = 1
NS_PA_DTYPE_F16 = 2
STATUS_BAD_BLOCK = 1
STATUS_SEQ_TOO_LONG = 2
STATUS_BAD_TILE = 4
TILE_COLUMNS = 128         # query columns of a prefill tile (NS_PA_TILE_COLUMNS): 128 // G tokens of G heads
PREFILL_MIN_QUERY = 2      # sequences with at least this many query tokens go by tile

EXPORTS = ("ns_pa_abi_version", "ns_pa_last_error", "ns_paged_attention_workspace_bytes",
           "ns_paged_attention_call_workspace", "ns_paged_attention")


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
        ("decode_tokens", ctypes.c_void_p),
        ("n_decode_tokens", ctypes.c_int32),
        ("prefill_tiles", ctypes.c_void_p),
        ("n_prefill_tiles", ctypes.c_int32),
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
    lib.ns_paged_attention_call_workspace.restype = ctypes.c_int
    lib.ns_paged_attention_call_workspace.argtypes = [ctypes.POINTER(NsPagedAttnArgs),
                                                      ctypes.POINTER(ctypes.c_uint64),
                                                      ctypes.POINTER(ctypes.c_uint64)]
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


def plan_tiles(seq_lens, query_start_loc, query_lens, num_heads_q: int, num_kv_heads: int):
    """Host plan of a batch with prefill chunks: (tiles, decode tokens) as int32 numpy arrays.
    Each sequence with at least PREFILL_MIN_QUERY query tokens is cut into tiles of
    TILE_COLUMNS // G consecutive tokens, (sequence, first token, count) each; every other query
    token is listed for the per-token kernel."""
    import numpy as np

    ql = np.asarray(query_lens, dtype=np.int64)
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    bq = TILE_COLUMNS // (num_heads_q // num_kv_heads)
    tiles, tokens = [], []
    for s in range(ql.size):
        q, start = int(ql[s]), int(qsl[s])
        if q >= PREFILL_MIN_QUERY:
            for t in range(0, q, bq):
                tiles.append((s, start + t, min(bq, q - t)))
        elif q > 0:
            tokens.extend(range(start, start + q))
    return (np.asarray(tiles, dtype=np.int32).reshape(-1, 3), np.asarray(tokens, dtype=np.int32))


class PagedAttentionPlan:
    """The host plan of one batch layout, reusable by every layer's call of a step: the device
    lists of prefill tiles and per-token queries, and the layout's longest sequence and query.
    The reference's launcher reads the layout on every call (paged_attention_triton.py:120-121);
    with a plan the calls read nothing on the host."""

    def __init__(self, seq_lens, query_start_loc, query_lens, num_heads_q: int, num_kv_heads: int, device):
        import torch

        h_sl = np.asarray(seq_lens.cpu() if hasattr(seq_lens, "cpu") else seq_lens, dtype=np.int64).reshape(-1)
        h_qsl = np.asarray(query_start_loc.cpu() if hasattr(query_start_loc, "cpu") else query_start_loc,
                           dtype=np.int64).reshape(-1)
        h_ql = np.asarray(query_lens.cpu() if hasattr(query_lens, "cpu") else query_lens, dtype=np.int64).reshape(-1)
        self.num_heads_q, self.num_kv_heads = int(num_heads_q), int(num_kv_heads)
        self.total_q = int(h_ql.sum())
        self.max_seq_len = int(h_sl.max()) if h_sl.size else 0
        self.max_query_len = int(h_ql.max()) if h_ql.size else 0
        self.staged = None
        self.tokens = (0, 0)
        self.tiles = None
        if self.max_query_len >= PREFILL_MIN_QUERY:
            h_tiles, h_tokens = plan_tiles(h_sl, h_qsl, h_ql, num_heads_q, num_kv_heads)
            staged = torch.from_numpy(np.concatenate([h_tokens, h_tiles.reshape(-1)]).astype(np.int32))
            if torch.device(device).type == "cuda":
                staged = staged.pin_memory()
            self.staged = staged.to(device, non_blocking=True)
            # the per-token list starts the staged buffer (a valid address even when it is empty)
            self.tokens = (self.staged.data_ptr(), int(h_tokens.size))
            self.tiles = (self.staged.data_ptr() + 4 * int(h_tokens.size), int(h_tiles.shape[0]))


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
                        max_query_len: Optional[int] = None, plan: Optional[PagedAttentionPlan] = None,
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
    given.  ``max_query_len``: an upper bound of ``query_lens`` (1 for a decode step, which then
    takes the per-token kernel without reading the batch layout on the host).  ``plan``: a
    ``PagedAttentionPlan`` of this batch layout (then nothing is read on the host).  ``stream``: a ``torch.cuda.Stream`` or a raw HIP stream handle, default the current
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
    elif int(stream) == 0:
        # the null stream is torch's default stream (an ExternalStream of handle 0 is not it)
        s = torch.cuda.default_stream(dev)
    elif int(stream) == torch.cuda.current_stream(dev).cuda_stream:
        s = torch.cuda.current_stream(dev)
    else:
        s = torch.cuda.ExternalStream(int(stream), device=dev)
    with torch.cuda.stream(s):
        return _paged_attention_on(lib, s, query, k_cache, v_cache, block_tables, seq_lens, query_start_loc,
                                   query_lens, scale, block_size, max_seq_len, max_query_len, plan, out,
                                   workspace, counters, status)


def _paged_attention_on(lib, s, query, k_cache, v_cache, block_tables, seq_lens, query_start_loc, query_lens,
                        scale, block_size, max_seq_len, max_query_len, plan, out, workspace, counters, status):
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
    # prefill tiles: 16-bit types, unless the caller declares a decode step
    tiles = tokens = None
    if plan is not None:
        if plan.total_q != total_q or plan.num_heads_q != hq or plan.num_kv_heads != hkv:
            raise PagedAttentionError("the plan was made for another batch layout or head layout")
        if max_seq_len is None:
            max_seq_len = plan.max_seq_len
    elif query.dtype != torch.float32 and (max_query_len is None or max_query_len >= PREFILL_MIN_QUERY):
        plan = PagedAttentionPlan(sl, qsl, ql, hq, hkv, dev)   # one read of the batch layout
        if max_seq_len is None:
            max_seq_len = plan.max_seq_len
    if plan is not None and plan.tiles is not None and query.dtype != torch.float32:
        tokens, tiles = plan.tokens, plan.tiles
    if max_seq_len is None:
        max_seq_len = int(sl.max().item()) if num_seqs else 0
    if out is None:
        out = torch.empty_like(query)
    elif out.shape != query.shape or out.dtype != query.dtype or out.device != dev:
        raise PagedAttentionError("out must match query's shape, dtype and device")
    elif out.stride(-1) != 1:
        raise PagedAttentionError("out must have a unit head_dim stride")
    if status is not None and (status.dtype != torch.int32 or status.device != dev or status.numel() < 1):
        raise PagedAttentionError("status must be an int32 device tensor")
    a = NsPagedAttnArgs(
        query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), bt.data_ptr(), sl.data_ptr(),
        qsl.data_ptr(), ql.data_ptr(), status.data_ptr() if status is not None else None,
        None, 0, None,
        query.stride(0), query.stride(1), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2), out.stride(0), out.stride(1),
        bt.stride(0) if bt.dim() == 2 else 0,
        total_q, num_seqs, hq, hkv, d, bs, nb, bt.shape[1] if bt.dim() == 2 else 0, max_seq_len,
        _dtype_code(query.dtype), float(scale))
    if tiles is not None:
        a.decode_tokens, a.n_decode_tokens = tokens
        a.prefill_tiles, a.n_prefill_tiles = tiles
    need_b, need_c = ctypes.c_uint64(0), ctypes.c_uint64(0)
    _check(lib.ns_paged_attention_call_workspace(ctypes.byref(a), ctypes.byref(need_b), ctypes.byref(need_c)))
    need, ncount = int(need_b.value), int(need_c.value)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif need and workspace.numel() * workspace.element_size() < need:
        raise PagedAttentionError(
            f"workspace of {need} bytes needed, {workspace.numel() * workspace.element_size()} given (total_q "
            f"{total_q}, max_seq_len {max_seq_len}, {a.n_decode_tokens if tiles is not None else total_q} "
            f"per-token queries, {a.n_prefill_tiles if tiles is not None else 0} prefill tiles)")
    if need and counters is None:
        counters = counters_for(dev, ncount, s)
    elif need and (counters.dtype != torch.int32 or counters.device != dev or counters.numel() < ncount):
        raise PagedAttentionError(f"counters must be an int32 device tensor of at least {ncount} entries")
    if need:
        a.workspace, a.workspace_bytes, a.counters = workspace.data_ptr(), need, counters.data_ptr()
    _check(lib.ns_paged_attention(ctypes.byref(a), ctypes.c_void_p(int(s.cuda_stream))))
    return out


# the reference's name, so that nanoserve/model/attention.py:21 can import this module unchanged
paged_attention_triton = paged_attention_hip
