"""ctypes binding of the sampler's C ABI (include/ns_sampling.h).

Loads the in-tree ``libns_sampling.so`` built by ``build.py``.  There is no
fallback: if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libns_sampling.so")

NS_OK = 0
NS_DTYPE_F32 = 0
NS_DTYPE_BF16 = 1
NS_MAX_VOCAB = 262144
NS_MAX_HISTORY = 1 << 20   # per-row history limit (ids)
NS_LDS_HISTORY = 8192      # longest history the general per-row code keeps in LDS (longer: in the workspace)
NS_INFO_WORDS = 8
NS_MODE_AUTO = 0
NS_MODE_SEGMENTED = 1
NS_MODE_PER_ROW = 2
NS_KIND_GREEDY = 1      # row_kinds: greedy rows (temperature 0)
NS_KIND_SMALL_K = 2     # sampled rows with 1 <= top_k <= 64 and top_k < vocab
NS_KIND_OTHER = 4       # every other sampled row (top-k off or larger)
NS_DEBUG_STREAM, NS_DEBUG_WIDE, NS_DEBUG_GENERAL = 0, 1, 2   # ns_debug_scaled routines
NS_PENALTY_DIVIDE = 0       # penalty_rounding: score / p correctly rounded (torch on the CPU)
NS_PENALTY_RECIPROCAL = 1   # penalty_rounding: score * fl32(1 / p) (torch on a GPU)
PENALTY_ROUNDING = {"division": NS_PENALTY_DIVIDE, "reciprocal": NS_PENALTY_RECIPROCAL}
ABI_VERSION = 10

# exported symbols, as declared in include/ns_sampling.h
NS_NOALLOC_SCRATCH_BYTES = 80 << 20   # ns_sample_noalloc's device scratch per GPU
EXPORTS = ("ns_abi_version", "ns_sample", "ns_sample_noalloc", "ns_sample_lds_bytes", "ns_sample_workspace_bytes",
           "ns_hist_state_bytes",
           "ns_hist_assign", "ns_hist_append", "ns_seeded_uniforms", "ns_lm_head_bf16", "ns_lm_head_packed_bytes",
           "ns_lm_head_pack_bf16", "ns_lm_head_bf16_packed", "ns_debug_scaled", "ns_last_error")


class NsSampleArgs(ctypes.Structure):
    """Mirror of ``ns_sample_args`` (field order and types must match the header)."""

    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("n_sample", ctypes.c_int32),
        ("n_rows_total", ctypes.c_int64),
        ("vocab", ctypes.c_int64),
        ("row_stride", ctypes.c_int64),
        ("sample_idx", ctypes.c_void_p),
        ("temperature", ctypes.c_void_p),
        ("top_k", ctypes.c_void_p),
        ("top_p", ctypes.c_void_p),
        ("rep_penalty", ctypes.c_void_p),
        ("hist_offsets", ctypes.c_void_p),
        ("hist_ids", ctypes.c_void_p),
        ("max_hist", ctypes.c_int32),
        ("uniforms", ctypes.c_void_p),
        ("out_ids", ctypes.c_void_p),
        ("out_probs", ctypes.c_void_p),
        ("out_info", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("mode", ctypes.c_int32),
        ("row_kinds", ctypes.c_uint32),
        ("hist_state", ctypes.c_void_p),
        ("hist_slot", ctypes.c_void_p),
        ("hist_n_slots", ctypes.c_int32),
        ("hist_capacity", ctypes.c_int32),
        ("hist_append", ctypes.c_int32),
        ("hist_overflow", ctypes.c_void_p),
        ("penalty_rounding", ctypes.c_int32),
        ("rep_penalty_recip", ctypes.c_void_p),
    ]


class SamplerLibraryError(RuntimeError):
    pass


_LIB: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the native library once; raise if it is missing or incompatible."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise SamplerLibraryError(
            f"native sampler library not found at {path}; build it with build.py (hipcc, gfx950)")
    lib = ctypes.CDLL(path)
    lib.ns_abi_version.restype = ctypes.c_int
    lib.ns_abi_version.argtypes = []
    lib.ns_sample.restype = ctypes.c_int
    lib.ns_sample.argtypes = [ctypes.POINTER(NsSampleArgs), ctypes.c_void_p]
    lib.ns_sample_noalloc.restype = ctypes.c_int
    lib.ns_sample_noalloc.argtypes = [ctypes.POINTER(NsSampleArgs), ctypes.c_void_p]
    lib.ns_sample_lds_bytes.restype = ctypes.c_int
    lib.ns_sample_lds_bytes.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32)]
    lib.ns_sample_workspace_bytes.restype = ctypes.c_int
    lib.ns_sample_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.POINTER(ctypes.c_uint64)]
    lib.ns_hist_state_bytes.restype = ctypes.c_int
    lib.ns_hist_state_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)]
    lib.ns_hist_assign.restype = ctypes.c_int
    lib.ns_hist_assign.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                   ctypes.c_int32, ctypes.c_void_p]
    lib.ns_hist_append.restype = ctypes.c_int
    lib.ns_hist_append.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    lib.ns_debug_scaled.restype = ctypes.c_int
    lib.ns_debug_scaled.argtypes = [ctypes.POINTER(NsSampleArgs), ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
                                    ctypes.c_void_p]
    lib.ns_seeded_uniforms.restype = ctypes.c_int
    lib.ns_seeded_uniforms.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                       ctypes.c_void_p, ctypes.c_void_p]
    lib.ns_lm_head_bf16.restype = ctypes.c_int
    lib.ns_lm_head_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_void_p]
    lib.ns_lm_head_packed_bytes.restype = ctypes.c_int
    lib.ns_lm_head_packed_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)]
    lib.ns_lm_head_pack_bf16.restype = ctypes.c_int
    lib.ns_lm_head_pack_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_void_p, ctypes.c_void_p]
    lib.ns_lm_head_bf16_packed.restype = ctypes.c_int
    lib.ns_lm_head_bf16_packed.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_void_p,
                                           ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.ns_last_error.restype = ctypes.c_char_p
    lib.ns_last_error.argtypes = []
    v = lib.ns_abi_version()
    if v != ABI_VERSION:
        raise SamplerLibraryError(f"ABI version mismatch: library {v}, binding {ABI_VERSION}")
    _LIB = lib
    return lib


def last_error() -> str:
    return load().ns_last_error().decode(errors="replace")


def check(rc: int) -> None:
    if rc != NS_OK:
        raise SamplerLibraryError(f"ns_sample failed ({rc}): {last_error()}")


def lds_bytes(vocab: int, max_hist: int) -> int:
    out = ctypes.c_int32(0)
    check(load().ns_sample_lds_bytes(int(vocab), int(max_hist), ctypes.byref(out)))
    return int(out.value)


def workspace_bytes(n_sample: int, vocab: int, dtype: int, max_hist: int = 0) -> int:
    out = ctypes.c_uint64(0)
    check(load().ns_sample_workspace_bytes(int(n_sample), int(vocab), int(dtype), int(max_hist), ctypes.byref(out)))
    return int(out.value)


_WS = {}


def workspace_for(device, n_sample: int, vocab: int, dtype: int, max_hist: int = 0):
    """A cached zero-filled workspace tensor on ``device`` large enough for this call.

    One workspace per device, used on the current stream; it is regrown (and
    zero-filled again) when a call needs more.
    """
    import torch

    need = workspace_bytes(n_sample, vocab, dtype, max_hist)
    key = str(device)
    ws = _WS.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def row_kinds(temperature, top_k, vocab: int) -> int:
    """NS_KIND_* bits of the rows described by host arrays of temperatures and top_k values."""
    import numpy as np

    t = np.asarray(temperature)
    k = np.asarray(top_k)
    greedy = t == 0.0
    small = ~greedy & (k >= 1) & (k <= 64) & (k < vocab)
    kinds = 0
    if greedy.any():
        kinds |= NS_KIND_GREEDY
    if small.any():
        kinds |= NS_KIND_SMALL_K
    if (~greedy & ~small).any():
        kinds |= NS_KIND_OTHER
    return kinds


def _ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def aligned_rows(logits, sample_idx):
    """``(logits, sample_idx)`` with every row starting on a 16-byte boundary.

    The kernels read rows in 16-byte chunks, so the C ABI rejects misaligned
    rows (NS_ERR_ALIGN).  Vocabularies whose row size is not a multiple of 16
    bytes (an odd fp32 vocab such as 50257) and misaligned views are copied
    here into rows padded to a multiple of 16 bytes: only the sampled rows
    when ``sample_idx`` is given.  The gather reads clamped indices, so an
    index outside the tensor reads nothing out of bounds; the returned
    ``sample_idx`` is the identity for valid rows and -1 for the others, which
    the kernels report as bad rows (id -1) as they do without the copy.
    Aligned inputs, every vocab used by the benchmarks among them, are passed
    through.
    """
    import torch

    esz = logits.element_size()
    if logits.data_ptr() % 16 == 0 and (logits.stride(0) * esz) % 16 == 0:
        return logits, sample_idx
    new_idx = None
    if sample_idx is None:
        rows = logits
    else:
        n = int(logits.shape[0])
        idx = sample_idx.to(torch.int64)
        valid = (idx >= 0) & (idx < n)
        rows = logits.index_select(0, idx.clamp(0, max(n - 1, 0)))
        new_idx = torch.where(valid, torch.arange(idx.numel(), device=idx.device, dtype=torch.int64),
                              torch.full_like(idx, -1))
    V = int(rows.shape[1])
    per = 16 // esz
    padded = torch.empty((int(rows.shape[0]), (V + per - 1) // per * per), dtype=rows.dtype, device=rows.device)
    padded[:, :V].copy_(rows)
    return padded[:, :V], new_idx


def penalty_reciprocals(penalties):
    """fl32(1 / p) of float64 penalties, the reciprocal rounded once: what torch on a GPU
    multiplies by for ``score / p`` with a Python float p (sampler.py:37)."""
    import numpy as np

    p = np.asarray(penalties, dtype=np.float64)
    with np.errstate(divide="ignore"):
        return (1.0 / p).astype(np.float32)


def sample_raw(logits, temperature, top_k, top_p, rep_penalty, uniforms, out_ids, *, sample_idx=None,
               hist_offsets=None, hist_ids=None, max_hist: int = 0, out_probs=None, out_info=None,
               stream=None, workspace="auto", mode: int = NS_MODE_AUTO, row_kinds: int = 0,
               hist_state=None, hist_slot=None, hist_append: bool = False, hist_overflow=None,
               debug_scaled=None, penalty_rounding: int = NS_PENALTY_DIVIDE, rep_penalty_recip=None) -> None:
    """Launch ``ns_sample`` on device tensors (no copies, no synchronisation).

    logits: (N, V) float32 or bfloat16 CUDA tensor with unit stride in the last dim.
    temperature/top_p/rep_penalty/uniforms: (B,) float32; top_k: (B,) int32;
    sample_idx: (B,) int64 or None; hist_offsets: (B+1,) int32; hist_ids: int32;
    out_ids: (B,) int64; out_probs: (B, V) float32 or None; out_info: (B, 8) int32 or None.
    workspace: "auto" (a cached per-device workspace), a uint8 CUDA tensor, or None (every row
    takes the one-workgroup-per-row kernel).  row_kinds: NS_KIND_* bits of the rows present
    (see ``row_kinds``), 0 when unknown.  hist_state / hist_slot: device-resident histories
    (a ``HistoryState`` and the (B,) int32 slot of each row, -1 for none) instead of
    hist_offsets / hist_ids.  hist_append: the kernels also append each row's sampled id to
    its slot (HistoryState.append fused into the call; the rows name distinct slots);
    hist_overflow: a (1,) int32 tensor counting full slots, or None.
    debug_scaled: a pair (formula, out) with out a (B, >= V) float32 tensor of unit stride
    along V: instead of sampling, ``ns_debug_scaled`` writes each row's penalized,
    temperature-scaled logits there, computed by routine ``formula`` (NS_DEBUG_*).
    penalty_rounding: NS_PENALTY_DIVIDE (score / p correctly rounded, as torch on the CPU) or
    NS_PENALTY_RECIPROCAL (score * rep_penalty_recip[r], as torch on a GPU);
    rep_penalty_recip: (B,) float32, each row's fl32(1 / p) from the float64 penalty (see
    ``penalty_reciprocals``), needed with NS_PENALTY_RECIPROCAL.
    """
    import torch

    lib = load()
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a 2-D tensor with unit stride along the vocabulary")
    if logits.dtype == torch.float32:
        dt = NS_DTYPE_F32
    elif logits.dtype == torch.bfloat16:
        dt = NS_DTYPE_BF16
    else:
        raise TypeError(f"logits dtype {logits.dtype} not supported (float32 or bfloat16)")
    B = int(out_ids.shape[0])
    logits, sample_idx = aligned_rows(logits, sample_idx)
    a = NsSampleArgs()
    a.logits = _ptr(logits)
    a.dtype = dt
    a.n_sample = B
    a.n_rows_total = int(logits.shape[0])
    a.vocab = int(logits.shape[1])
    a.row_stride = int(logits.stride(0))
    a.sample_idx = _ptr(sample_idx)
    a.temperature = _ptr(temperature)
    a.top_k = _ptr(top_k)
    a.top_p = _ptr(top_p)
    a.rep_penalty = _ptr(rep_penalty)
    a.hist_offsets = _ptr(hist_offsets)
    a.hist_ids = _ptr(hist_ids)
    a.max_hist = int(max_hist)
    a.uniforms = _ptr(uniforms)
    a.out_ids = _ptr(out_ids)
    a.out_probs = _ptr(out_probs)
    a.out_info = _ptr(out_info)
    if isinstance(workspace, str) and workspace == "auto":
        workspace = workspace_for(logits.device, B, a.vocab, dt,
                                  max_hist if (hist_offsets is not None or hist_state is not None) else 0)
    if workspace is not None:
        a.workspace = _ptr(workspace)
        a.workspace_bytes = int(workspace.numel() * workspace.element_size())
    a.mode = int(mode)
    a.row_kinds = int(row_kinds)
    a.penalty_rounding = int(penalty_rounding)
    a.rep_penalty_recip = _ptr(rep_penalty_recip)
    if hist_state is not None:
        if hist_offsets is not None or hist_ids is not None:
            raise ValueError("hist_state excludes hist_offsets / hist_ids")
        a.hist_state = _ptr(hist_state.buffer)
        a.hist_slot = _ptr(hist_slot)
        a.hist_n_slots = int(hist_state.n_slots)
        a.hist_capacity = int(hist_state.capacity)
    if hist_append:
        if hist_state is None:
            raise ValueError("hist_append needs hist_state")
        a.hist_append = 1
        a.hist_overflow = _ptr(hist_overflow)
    if stream is None:
        stream = torch.cuda.current_stream(logits.device)
    if debug_scaled is not None:
        formula, out = debug_scaled
        if out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1 or int(out.shape[0]) < B:
            raise ValueError("debug output must be a (B, >= V) float32 tensor with unit stride along V")
        check(lib.ns_debug_scaled(ctypes.byref(a), int(formula), _ptr(out), int(out.stride(0)),
                                  ctypes.c_void_p(int(stream.cuda_stream))))
        return
    check(lib.ns_sample(ctypes.byref(a), ctypes.c_void_p(int(stream.cuda_stream))))


class PackedLmHead:
    """An lm_head weight ((V, H) bf16) packed once by ns_lm_head_pack_bf16 into contiguous
    256 x 64 tiles, for ``lm_head_bf16``: the same logits, with the weight streamed at
    close to the HBM rate.  Holds its own device buffer; the weight itself is not kept."""

    def __init__(self, weight, stream=None):
        import torch

        if weight.dtype != torch.bfloat16 or weight.dim() != 2 or weight.stride(1) != 1:
            raise ValueError("weight must be a (V, H) bfloat16 tensor with unit stride along H")
        self.n, self.k = int(weight.shape[0]), int(weight.shape[1])
        nbytes = ctypes.c_uint64(0)
        check(load().ns_lm_head_packed_bytes(self.n, self.k, ctypes.byref(nbytes)))
        self.buffer = torch.empty(int(nbytes.value), dtype=torch.uint8, device=weight.device)
        if stream is None:
            stream = torch.cuda.current_stream(weight.device)
        check(load().ns_lm_head_pack_bf16(_ptr(weight), int(weight.stride(0)), self.n, self.k, _ptr(self.buffer),
                                          ctypes.c_void_p(int(stream.cuda_stream))))

    @property
    def shape(self):
        return (self.n, self.k)


def lm_head_bf16(hidden, weight, rows=None, out=None, stream=None):
    """bf16 logits = hidden[rows] @ weight.T through ns_lm_head_bf16 (fp32 accumulation).

    hidden: (N, H) bf16 with unit stride along H; weight: (V, H) bf16, the lm_head /
    tied-embedding layout, or a ``PackedLmHead`` of it; rows: optional (B,) int64 device
    tensor of hidden rows (the step's sample positions), else every row; out: optional
    (B, V) bf16 tensor.
    """
    import torch

    packed = isinstance(weight, PackedLmHead)
    if hidden.dtype != torch.bfloat16 or (not packed and weight.dtype != torch.bfloat16):
        raise ValueError("hidden and weight must be bfloat16")
    if hidden.dim() != 2 or len(weight.shape) != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"shapes {tuple(hidden.shape)} and {tuple(weight.shape)} do not match (N, H) x (V, H)")
    if hidden.stride(1) != 1 or (not packed and weight.stride(1) != 1):
        raise ValueError("hidden and weight need unit stride along the hidden dimension")
    if rows is not None and (rows.dtype != torch.int64 or rows.dim() != 1 or not rows.is_contiguous()):
        raise ValueError("rows must be a contiguous (B,) int64 tensor")
    m = int(rows.numel()) if rows is not None else int(hidden.shape[0])
    n, k = int(weight.shape[0]), int(weight.shape[1])
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=hidden.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (m, n) or out.stride(1) != 1:
        raise ValueError(f"out must be a (B, V) = ({m}, {n}) bf16 tensor with unit column stride")
    if stream is None:
        stream = torch.cuda.current_stream(hidden.device)
    sh = ctypes.c_void_p(int(stream.cuda_stream))
    rp = _ptr(rows) if rows is not None else 0
    if packed:
        check(load().ns_lm_head_bf16_packed(_ptr(hidden), int(hidden.stride(0)), int(hidden.shape[0]), rp,
                                            _ptr(weight.buffer),
                                            int(weight.buffer.numel()), _ptr(out), int(out.stride(0)), m, n, k, sh))
    else:
        check(load().ns_lm_head_bf16(_ptr(hidden), int(hidden.stride(0)), int(hidden.shape[0]), rp, _ptr(weight),
                                     int(weight.stride(0)),
                                     _ptr(out), int(out.stride(0)), m, n, k, sh))
    return out


def seeded_uniforms(seeds, steps, rows, out, stream=None) -> None:
    """out[rows[j]] = the Philox4x32-10 uniform of (seeds[j], steps[j]) (ns_seeded_uniforms).

    ``seeds``: host sequence of Python ints (taken modulo 2^64); ``steps``: host sequence of
    history lengths; ``rows``: host sequence of row indices into ``out`` ((B,) float32 device
    tensor).  The three arrays travel to the device in one copy.
    """
    import numpy as np
    import torch

    n = len(rows)
    if n == 0:
        return
    if not (len(seeds) == len(steps) == n):
        raise ValueError("seeds, steps and rows must have one entry per seeded row")
    for r in rows:
        if not 0 <= int(r) < out.numel():
            raise ValueError("seeded row index outside the uniforms tensor")
    host = np.empty(3 * n, dtype=np.int64)
    host[:n] = np.array([int(x) & 0xFFFFFFFFFFFFFFFF for x in seeds], dtype=np.uint64).view(np.int64)
    host[n:2 * n] = np.asarray(steps, dtype=np.int64)
    host[2 * n:] = np.asarray(rows, dtype=np.int64)
    dev = torch.from_numpy(host).to(out.device)
    rows32 = dev[2 * n:].to(torch.int32)
    if stream is None:
        stream = torch.cuda.current_stream(out.device)
    check(load().ns_seeded_uniforms(_ptr(dev), _ptr(dev) + 8 * n, _ptr(rows32), n, _ptr(out),
                                    ctypes.c_void_p(int(stream.cuda_stream))))


def hist_state_bytes(n_slots: int, capacity: int) -> int:
    out = ctypes.c_uint64(0)
    check(load().ns_hist_state_bytes(int(n_slots), int(capacity), ctypes.byref(out)))
    return int(out.value)


class HistoryState:
    """Device-resident histories: ``n_slots`` request slots of up to ``capacity`` token ids.

    The buffer is the layout ``ns_hist_state_bytes`` describes (lengths, then ids), zero
    filled, so every slot starts empty.  ``assign`` sets a slot (a request's prompt) and
    ``append`` adds one sampled token per row; both run on the given stream.
    """

    def __init__(self, device, n_slots: int, capacity: int):
        import torch

        self.n_slots = int(n_slots)
        self.capacity = int(capacity)
        self.buffer = torch.zeros(hist_state_bytes(self.n_slots, self.capacity), dtype=torch.uint8, device=device)
        self.overflow = torch.zeros(1, dtype=torch.int32, device=device)

    def assign(self, slot: int, ids, stream=None) -> None:
        """Slot ``slot`` holds ``ids`` ((n,) int32 device tensor, n <= capacity) from now on."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.buffer.device)
        n = int(ids.numel()) if ids is not None else 0
        check(load().ns_hist_assign(_ptr(self.buffer), self.n_slots, self.capacity, int(slot),
                                    _ptr(ids) if n > 0 else 0, n, ctypes.c_void_p(int(stream.cuda_stream))))

    def append(self, slots, token_ids, stream=None) -> None:
        """token_ids[r] joins slot slots[r] ((B,) int32 and (B,) int64 device tensors)."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.buffer.device)
        check(load().ns_hist_append(_ptr(self.buffer), self.n_slots, self.capacity, _ptr(slots), _ptr(token_ids),
                                    int(slots.numel()), _ptr(self.overflow),
                                    ctypes.c_void_p(int(stream.cuda_stream))))
