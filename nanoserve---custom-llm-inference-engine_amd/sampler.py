"""Batched token sampler on MI355X: the host mirror of NanoServe's ``Sampler``.

Same class, constructor and ``sample()`` surface as the reference
(nanoserve/scheduler/sampler.py:17-29), so the engine's call at
nanoserve/engine/engine.py:247-249 and the ``.tolist()`` hand-off to
``Scheduler.update_with_sampled`` (scheduler.py:264-284) work unchanged.
All arithmetic of sampler.py:31-89 runs in one HIP kernel launch
(``ns_sample``, include/ns_sampling.h); this module only packs the per-row
parameters and histories into device arrays.

Additions, all keyword-only and optional:

* ``sample_indices``: rows of ``logits`` to sample (the scheduler's
  ``sample_indices``, scheduler.py:240-246), so the caller can pass the whole
  flat logits tensor and skip the ``index_select`` at engine.py:235.
* ``uniforms``: one float32 in [0, 1) per sampled row for the inverse-CDF
  draw.  When omitted, a row whose ``SamplingParams.seed`` is set draws a
  Philox4x32-10 uniform keyed by the seed and counted by its history length
  (``ns_seeded_uniforms``: the same seed and history give the same token on
  every call); the other rows draw from ``generators[i]`` where given (the
  reference accepts ``generators`` and ``seed`` but uses neither,
  sampler.py:26, config.py:79) and from the global CUDA generator otherwise.
* ``logits`` may be float32 or bfloat16 (bf16 is read directly; no
  ``.float()`` copy as at engine.py:236).
* ``device_histories`` / ``history_requests``: histories kept on the device
  (``DeviceHistories``) instead of the per-step ``history_token_ids`` lists.
  The engine rebuilds prompt + output ids for every request and step
  (engine.py:242-246) and the reference copies them to the device each call
  (sampler.py:34); here each request's ids are copied once when it starts and
  every sampled token is appended on the device by the kernel that draws it.
* ``async_ids``: return a ``SampledIds`` handle instead of the tensor.  Its ids
  are copied into a pinned host buffer of the sampler's ``ReadbackRing`` behind
  an event on the same stream, so ``.tolist()`` (engine.py:250) waits only when
  the engine reads them and the next step's host work can run meanwhile.

Differences that the engine cannot observe: the caller's logits are not
modified in place (the reference's penalty writes into them, sampler.py:38,
and engine.py never reads them again); the draw is an inverse CDF against the
uniforms instead of ``torch.multinomial``'s exponential race (sampler.py:87),
which is the same distribution.
"""
from __future__ import annotations

import itertools
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .config import SamplingParams

_I32_MAX = 2**31 - 1


def effective_temperature(t: float) -> float:
    """sampler.py:42: ``max(t, 1e-6) if t > 0 else 1.0`` (greedy when t == 0)."""
    return max(t, 1e-6) if t > 0 else 1.0


class PackedRows:
    """Per-row parameters and CSR histories (or device history slots) packed for one call."""

    def __init__(self, params: Sequence[SamplingParams], histories: Sequence, vocab: int,
                 slots: Optional[np.ndarray] = None, slot_max_hist: int = 0, penalty_rounding: str = "division"):
        B = len(params)
        # the four numeric fields of every row in one pass (float64 holds each float field
        # exactly and top_k exactly below 2^53; larger top_k values clamp the same way)
        try:
            f4 = np.fromiter(itertools.chain.from_iterable(
                (p.temperature, p.top_k, p.top_p, p.repetition_penalty) for p in params), dtype=np.float64,
                count=4 * B).reshape(B, 4)
        except (TypeError, ValueError, OverflowError):
            f4 = None
        if f4 is not None and np.isfinite(f4[:, 1]).all():
            t64, rp64 = f4[:, 0], f4[:, 3]
            topk = np.clip(np.trunc(f4[:, 1]), -1, _I32_MAX).astype(np.int32)
            topp = f4[:, 2].astype(np.float32)
        else:
            # the field-by-field conversions (and their errors: a top_k that is no integer)
            t64 = np.asarray([float(p.temperature) for p in params], dtype=np.float64).reshape(B)
            topk = np.asarray([min(max(int(p.top_k), -1), _I32_MAX) for p in params], dtype=np.int32).reshape(B)
            topp = np.asarray([float(p.top_p) for p in params], dtype=np.float64).reshape(B).astype(np.float32)
            rp64 = np.asarray([float(p.repetition_penalty) for p in params], dtype=np.float64).reshape(B)
        # greedy rows are encoded as temperature 0 (sampler.py:47-50); others carry the
        # effective float32 temperature, max(t, 1e-6) if t > 0 else 1 (sampler.py:41-46)
        temp = np.where(t64 == 0.0, 0.0, np.where(t64 > 0.0, np.maximum(t64, 1e-6), 1.0)).astype(np.float32)
        pen = rp64.astype(np.float32)
        lens = np.zeros(B, dtype=np.int64)
        hist_rows = [None] * B
        # every row's history length (the seeded uniform's counter), penalized or not
        self.history_lengths = [0] * B
        self.seeds = [p.seed for p in params]
        self.vocab = int(vocab)
        if histories is not None:
            for i in range(min(B, len(histories))):
                h = histories[i]
                self.history_lengths[i] = len(h) if h is not None else 0
                # only penalised rows index their history (sampler.py:33)
                if rp64[i] != 1.0 and len(h) > 0:
                    a = np.asarray(h, dtype=np.int64)
                    if a.size and (a.min() < 0 or a.max() >= vocab):
                        bad = int(a[(a < 0) | (a >= vocab)][0])
                        raise IndexError(f"history token id {bad} out of range for vocab {vocab} (row {i})")
                    hist_rows[i] = a.astype(np.int32)
                    lens[i] = a.size
        self.batch = B
        self.row_kinds = _lib.row_kinds(temp, topk, vocab)
        self.temperature = temp
        self.top_k = topk
        self.top_p = topp
        self.penalty = pen
        # the reciprocal penalty multiplies by fl32(1 / p), p the float64 parameter (sampler.py:37
        # as torch computes it on a GPU)
        self.penalty_rounding = _lib.PENALTY_ROUNDING[penalty_rounding]
        self.penalty_recip = (_lib.penalty_reciprocals(rp64) if penalty_rounding == "reciprocal" else None)
        self.max_hist = int(lens.max()) if B else 0
        self.slots = None
        if slots is not None:
            self.slots = np.ascontiguousarray(slots, dtype=np.int32)
            self.max_hist = int(slot_max_hist)
        if self.max_hist > _lib.NS_MAX_HISTORY:
            raise ValueError(f"history of {self.max_hist} tokens exceeds the supported {_lib.NS_MAX_HISTORY}")
        if self.max_hist > 0 and self.slots is None:
            offs = np.zeros(B + 1, dtype=np.int32)
            np.cumsum(lens, out=offs[1:])
            ids = np.concatenate([r for r in hist_rows if r is not None]) if any(
                r is not None for r in hist_rows) else np.zeros(0, dtype=np.int32)
            self.hist_offsets = offs
            self.hist_ids = ids.astype(np.int32, copy=False)
        else:
            self.hist_offsets = None
            self.hist_ids = None

    def to_device(self, device):
        """One host-to-device copy of everything (a single int32 staging buffer)."""
        B = self.batch
        nh = 0 if self.hist_ids is None else int(self.hist_ids.size)
        no = 0 if self.hist_offsets is None else B + 1
        if self.slots is not None:   # device histories: the slot of each row in place of the CSR
            no, nh = B, 0
        nr = B if self.penalty_recip is not None else 0
        buf = np.empty(4 * B + no + nh + nr, dtype=np.int32)
        buf[0:B] = self.temperature.view(np.int32)
        buf[B:2 * B] = self.top_k
        buf[2 * B:3 * B] = self.top_p.view(np.int32)
        buf[3 * B:4 * B] = self.penalty.view(np.int32)
        if self.slots is not None:
            buf[4 * B:5 * B] = self.slots
        elif no:
            buf[4 * B:4 * B + no] = self.hist_offsets
            buf[4 * B + no:4 * B + no + nh] = self.hist_ids
        if nr:
            buf[4 * B + no + nh:] = self.penalty_recip.view(np.int32)
        host = torch.from_numpy(buf)
        if torch.device(device).type == "cuda":
            host = host.pin_memory()
        dev = host.to(device, non_blocking=True)
        out = {
            "temperature": dev[0:B].view(torch.float32),
            "top_k": dev[B:2 * B],
            "top_p": dev[2 * B:3 * B].view(torch.float32),
            "rep_penalty": dev[3 * B:4 * B].view(torch.float32),
            "hist_offsets": dev[4 * B:4 * B + no] if no and self.slots is None else None,
            "hist_ids": dev[4 * B + no:4 * B + no + nh] if no and self.slots is None else None,
            "hist_slot": dev[4 * B:5 * B] if self.slots is not None else None,
            "rep_penalty_recip": dev[4 * B + no + nh:].view(torch.float32) if nr else None,
        }
        return out


class _ReadbackSlot:
    """One pinned host buffer and its event, reused by successive ``SampledIds``."""

    __slots__ = ("host", "event", "owner")

    def __init__(self, n: int):
        self.host = torch.empty(max(int(n), 256), dtype=torch.int64, pin_memory=True)
        self.event = torch.cuda.Event()
        self.owner = None


class ReadbackRing:
    """A fixed ring of pinned host buffers and events for ``async_ids``: nothing is allocated
    per call once the ring has filled (a buffer grows only for a larger batch).

    A slot is reused ``depth`` calls later.  If its previous handle has not been read by then,
    that handle first copies its ids out of the slot (waiting for its own copy), so a handle
    stays readable however long it is kept; an engine that reads each step's ids before the
    step after next never waits there.
    """

    def __init__(self, depth: int = 4):
        if depth < 1:
            raise ValueError("depth must be at least 1")
        self.depth = int(depth)
        self._slots: List[_ReadbackSlot] = []
        self._next = 0

    def readback(self, out: torch.Tensor) -> "SampledIds":
        """Queue the copy of ``out`` (int64, on the GPU) into the next slot behind an event on
        the current stream of ``out``'s device."""
        n = int(out.numel())
        if len(self._slots) < self.depth:
            self._slots.append(_ReadbackSlot(n))
            slot = self._slots[-1]
        else:
            slot = self._slots[self._next]
            self._next = (self._next + 1) % self.depth
            if slot.owner is not None:
                slot.owner._detach()
            if slot.host.numel() < n:
                slot.host = torch.empty(n, dtype=torch.int64, pin_memory=True)
        slot.host[:n].copy_(out, non_blocking=True)
        slot.event.record(torch.cuda.current_stream(out.device))
        h = SampledIds(out, slot, n)
        slot.owner = h
        return h


class SampledIds:
    """Sampled ids on their way to the host: ``.tolist()`` waits for the copy.

    ``tensor`` is the (B,) int64 device result (for further GPU work); ``ready()``
    tells without waiting whether the host copy has landed.
    """

    def __init__(self, tensor: torch.Tensor, slot: "_ReadbackSlot", n: int):
        self.tensor = tensor
        self._slot = slot
        self._n = n
        self._ids: Optional[List[int]] = None

    def _detach(self) -> None:
        """Copy the ids out of the ring slot before the slot is reused."""
        if self._ids is None:
            self._slot.event.synchronize()
            self._ids = self._slot.host[:self._n].tolist()
        self._slot = None

    def ready(self) -> bool:
        return self._ids is not None or bool(self._slot.event.query())

    def tolist(self) -> List[int]:
        if self._ids is None:
            self._slot.event.synchronize()
            self._ids = self._slot.host[:self._n].tolist()
        return list(self._ids)

    def __len__(self) -> int:
        return self._n


class DeviceHistories:
    """Per-request token histories kept on the device across ``sample`` calls.

    ``open(request_id, prompt_ids)`` gives a request a slot and copies its prompt
    once; ``Sampler.sample(..., device_histories=self, history_requests=ids)``
    reads each row's history from its request's slot and appends the sampled
    token to it on the device (the lists engine.py:242-246 rebuilds every step and
    sampler.py:34 copies to the device).  ``close(request_id)`` frees the slot.
    ``capacity`` bounds prompt + generated tokens per request: by default 8192,
    the reference's max_model_len; at most the sampler's per-row limit of 2^20.
    """

    def __init__(self, device, max_requests: int, capacity: int = _lib.NS_LDS_HISTORY):
        self.device = torch.device(device)
        self.state = _lib.HistoryState(self.device, max_requests, capacity)
        self.capacity = int(capacity)
        self._slot = {}
        self._free = list(range(int(max_requests) - 1, -1, -1))
        self._len = np.zeros(int(max_requests), dtype=np.int64)

    def open(self, request_id, prompt_ids: Sequence[int]) -> int:
        if request_id in self._slot:
            raise KeyError(f"request {request_id!r} already has a history slot")
        if not self._free:
            raise RuntimeError("no free history slot (raise max_requests)")
        ids = np.asarray(prompt_ids, dtype=np.int64).reshape(-1)
        if ids.size > self.capacity:
            raise ValueError(f"prompt of {ids.size} tokens exceeds the history capacity {self.capacity}")
        slot = self._free.pop()
        dev_ids = torch.from_numpy(ids.astype(np.int32)).to(self.device) if ids.size else None
        self.state.assign(slot, dev_ids)
        self._slot[request_id] = slot
        self._len[slot] = ids.size
        return slot

    def close(self, request_id) -> None:
        slot = self._slot.pop(request_id)
        self._len[slot] = 0
        self._free.append(slot)

    def length(self, request_id) -> int:
        return int(self._len[self._slot[request_id]])

    def slots(self, request_ids: Sequence) -> np.ndarray:
        return np.fromiter((self._slot[r] for r in request_ids), dtype=np.int32, count=len(request_ids))

    def _check_room(self, slots: np.ndarray) -> None:
        """Raise before any launch if a slot cannot take one more token."""
        full = self._len[slots] >= self.capacity
        if full.any():
            raise RuntimeError(f"history slot {int(slots[full][0])} is full ({self.capacity} tokens)")

    def _appended(self, slots: np.ndarray) -> None:
        """Count one appended token per slot, once the append has been issued."""
        self._len[slots] += 1


class Sampler:
    """Drop-in for nanoserve.scheduler.sampler.Sampler (sampler.py:17-19).

    ``penalty_rounding`` (keyword-only): how the repetition penalty's ``score / p``
    (sampler.py:37) rounds.  ``"division"`` (default): correctly rounded, as torch computes it on
    the CPU and as the source line reads.  ``"reciprocal"``: ``score * fl32(1 / p)`` (the float64
    reciprocal rounded once), as torch computes it on a GPU, the reference's default device
    (config.py:63).
    """

    def __init__(self, device: torch.device, *, penalty_rounding: str = "division"):
        self.device = device
        if penalty_rounding not in _lib.PENALTY_ROUNDING:
            raise ValueError(f"penalty_rounding must be one of {sorted(_lib.PENALTY_ROUNDING)}")
        self.penalty_rounding = penalty_rounding
        self._ring: Optional[ReadbackRing] = None   # pinned buffers and events of async_ids
        _lib.load()  # fail loudly at construction if the native library is missing

    def sample(
        self,
        logits: torch.Tensor,                # (num_seqs, vocab_size), or (N, vocab) with sample_indices
        sampling_params_list: List[SamplingParams],
        history_token_ids: List[List[int]],  # for repetition penalty
        generators: Optional[List[Optional[torch.Generator]]] = None,
        *,
        sample_indices: Optional[torch.Tensor] = None,
        uniforms: Optional[torch.Tensor] = None,
        return_probs: bool = False,
        device_histories: Optional[DeviceHistories] = None,
        history_requests: Optional[Sequence] = None,
        async_ids: bool = False,
    ):
        """Sample one token per row; returns an int64 tensor on ``logits.device``.

        ``sampling_params_list`` may also be the ``PackedRows`` of ``pack()`` (its
        ``history_token_ids`` and ``history_requests`` were taken there).
        With ``return_probs=True`` returns ``(ids, probs)`` where ``probs`` holds the
        final (B, V) probabilities of every non-greedy row (sampler.py:76-80).  With
        ``device_histories`` the histories are those of ``history_requests`` (one request
        per row, each at most once) and ``history_token_ids`` is ignored; the sampled
        tokens are appended to them.  With ``async_ids=True`` the result is a
        ``SampledIds`` handle (its ``.tolist()`` waits for the host copy), and
        ``(SampledIds, probs)`` with ``return_probs``.
        """
        if logits.device.type != "cuda":
            raise RuntimeError("the MI355X sampler needs logits on a GPU device")
        if logits.dim() != 2:
            raise ValueError("logits must be 2-D (rows, vocab)")
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        prepacked = isinstance(sampling_params_list, PackedRows)
        B = sampling_params_list.batch if prepacked else len(sampling_params_list)
        N, V = logits.shape
        if sample_indices is None and B != N:
            raise ValueError(f"{B} sampling params for {N} logits rows")
        dev = logits.device
        if prepacked:
            packed = sampling_params_list
            if packed.vocab != V:
                raise ValueError(f"rows packed for vocab {packed.vocab}, logits have {V}")
            if packed.penalty_rounding != _lib.PENALTY_ROUNDING[self.penalty_rounding]:
                raise ValueError("rows packed with another penalty rounding")
            if (packed.slots is not None) != (device_histories is not None):
                raise ValueError("rows packed with device histories need device_histories, and only they")
        slots = None
        if device_histories is not None:
            if prepacked:
                slots = packed.slots
            else:
                if history_requests is None or len(history_requests) != B:
                    raise ValueError("history_requests must name one request per sampled row")
                slots = device_histories.slots(history_requests)
                if len(set(slots.tolist())) != B:
                    raise ValueError("history_requests must name each request at most once")
            device_histories._check_room(slots)   # before any launch; counted once the append is issued
            max_hist = int(device_histories._len[slots].max()) if B else 0
            if prepacked:
                packed.max_hist = max_hist
            else:
                packed = PackedRows(sampling_params_list, None, V, slots=slots, slot_max_hist=max_hist,
                                    penalty_rounding=self.penalty_rounding)
        elif not prepacked:
            packed = PackedRows(sampling_params_list, history_token_ids, V, penalty_rounding=self.penalty_rounding)
        d = packed.to_device(dev)
        if sample_indices is not None:
            # a row outside the logits is refused here, as the reference's index_select
            # (engine.py:234) would raise: for a host list or CPU tensor without a sync; for a
            # device tensor only when device histories are appended to (one sync), since the
            # kernel gives such a row id -1 and appends nothing, which the host lengths must know
            if not (isinstance(sample_indices, torch.Tensor) and sample_indices.device.type == "cuda"):
                si = np.asarray(sample_indices.cpu() if isinstance(sample_indices, torch.Tensor) else sample_indices,
                                dtype=np.int64).reshape(-1)
                if si.size and (si.min() < 0 or si.max() >= N):
                    raise IndexError(f"sample index {int(si[(si < 0) | (si >= N)][0])} out of range for {N} rows")
                sample_indices = torch.from_numpy(si).to(dev)
            else:
                sample_indices = sample_indices.to(device=dev, dtype=torch.int64)
                if device_histories is not None and sample_indices.numel() > 0:
                    lo, hi = (int(v) for v in torch.aminmax(sample_indices))
                    if lo < 0 or hi >= N:
                        raise IndexError(f"sample index {lo if lo < 0 else hi} out of range for {N} rows")
            if sample_indices.numel() != B:
                raise ValueError("sample_indices must have one entry per sampling params")
        if uniforms is None:
            # rows whose request carries a seed draw a Philox uniform keyed by it and counted by
            # the history length (reproducible); the rest from ``generators`` or the device RNG
            seeded = [i for i, s in enumerate(packed.seeds) if s is not None]
            uniforms = self._draw_uniforms(B, dev, generators, skip=set(seeded))
            if seeded:
                if device_histories is not None:
                    steps = [int(device_histories._len[int(slots[i])]) for i in seeded]
                else:
                    steps = [packed.history_lengths[i] for i in seeded]
                _lib.seeded_uniforms([packed.seeds[i] for i in seeded], steps, seeded, uniforms)
        else:
            uniforms = uniforms.to(device=dev, dtype=torch.float32).contiguous()
            if uniforms.numel() != B:
                raise ValueError("uniforms must have one entry per sampled row")
        out = torch.empty(B, dtype=torch.int64, device=dev)
        probs = torch.empty((B, V), dtype=torch.float32, device=dev) if return_probs else None
        if B > 0:
            hs = device_histories.state if device_histories is not None else None
            _lib.sample_raw(logits, d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], uniforms, out,
                            sample_idx=sample_indices, hist_offsets=d["hist_offsets"], hist_ids=d["hist_ids"],
                            max_hist=packed.max_hist, out_probs=probs, row_kinds=packed.row_kinds,
                            hist_state=hs, hist_slot=d["hist_slot"], hist_append=hs is not None,
                            penalty_rounding=packed.penalty_rounding, rep_penalty_recip=d["rep_penalty_recip"])
            if hs is not None:
                device_histories._appended(slots)
        res = self._readback(out) if async_ids else out
        return (res, probs) if return_probs else res

    def pack(self, sampling_params_list: List[SamplingParams], history_token_ids=None, vocab: int = 0, *,
             device_histories: Optional[DeviceHistories] = None,
             history_requests: Optional[Sequence] = None) -> PackedRows:
        """The host half of ``sample``: the per-row parameters and histories packed for one call.

        ``sample(logits, packed, None, ...)`` takes the result in place of the parameters list
        (with the same ``device_histories``), so an engine can pack the next step's rows while
        the GPU samples this one and ``SampledIds`` carries its ids home (engine.py:238-250).
        """
        if device_histories is None:
            return PackedRows(sampling_params_list, history_token_ids, vocab, penalty_rounding=self.penalty_rounding)
        B = len(sampling_params_list)
        if history_requests is None or len(history_requests) != B:
            raise ValueError("history_requests must name one request per sampled row")
        slots = device_histories.slots(history_requests)
        if len(set(slots.tolist())) != B:
            raise ValueError("history_requests must name each request at most once")
        return PackedRows(sampling_params_list, None, vocab, slots=slots,
                          slot_max_hist=int(device_histories._len[slots].max()) if B else 0,
                          penalty_rounding=self.penalty_rounding)

    def _readback(self, out: torch.Tensor) -> SampledIds:
        """Copy ``out`` into the next pinned buffer of the sampler's ring behind an event on the
        current stream (no allocation once the ring has filled)."""
        if self._ring is None:
            self._ring = ReadbackRing()
        return self._ring.readback(out)

    @staticmethod
    def _draw_uniforms(B: int, dev, generators, skip=frozenset()) -> torch.Tensor:
        if len(skip) == B:
            return torch.empty(B, device=dev, dtype=torch.float32)   # every row seeded
        u = torch.rand(B, device=dev, dtype=torch.float32)
        if generators is not None:
            for i, g in enumerate(generators[:B]):
                if g is not None and i not in skip:
                    u[i] = torch.rand(1, generator=g, device=g.device, dtype=torch.float32).to(dev)[0]
        return u
