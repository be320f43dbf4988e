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
  are copied into pinned host memory behind an event on the same stream, so
  ``.tolist()`` (engine.py:250) waits only when the engine reads them and the
  next scheduler step can run meanwhile.

Differences that the engine cannot observe: the caller's logits are not
modified in place (the reference's penalty writes into them, sampler.py:38,
and engine.py never reads them again); the draw is an inverse CDF against the
uniforms instead of ``torch.multinomial``'s exponential race (sampler.py:87),
which is the same distribution.
"""
from __future__ import annotations

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
        # greedy rows are encoded as temperature 0 (sampler.py:47-50); others carry the
        # effective float32 temperature, max(t, 1e-6) if t > 0 else 1 (sampler.py:41-46)
        t64 = np.asarray([float(p.temperature) for p in params], dtype=np.float64).reshape(B)
        temp = np.where(t64 == 0.0, 0.0, np.where(t64 > 0.0, np.maximum(t64, 1e-6), 1.0)).astype(np.float32)
        topk = np.asarray([min(max(int(p.top_k), -1), _I32_MAX) for p in params], dtype=np.int32).reshape(B)
        topp = np.asarray([float(p.top_p) for p in params], dtype=np.float64).reshape(B).astype(np.float32)
        rp64 = np.asarray([float(p.repetition_penalty) for p in params], dtype=np.float64).reshape(B)
        pen = rp64.astype(np.float32)
        lens = np.zeros(B, dtype=np.int64)
        hist_rows = [None] * B
        if histories is not None:
            for i in range(min(B, len(histories))):
                h = histories[i]
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


class SampledIds:
    """Sampled ids on their way to the host: ``.tolist()`` waits for the copy.

    ``tensor`` is the (B,) int64 device result (for further GPU work); ``ready()``
    tells without waiting whether the host copy has landed.
    """

    def __init__(self, tensor: torch.Tensor, host: torch.Tensor, event):
        self.tensor = tensor
        self._host = host
        self._event = event

    def ready(self) -> bool:
        return bool(self._event.query())

    def tolist(self) -> List[int]:
        self._event.synchronize()
        return self._host.tolist()

    def __len__(self) -> int:
        return int(self.tensor.numel())


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
    the CPU and as the source line reads.  ``"reciprocal"``: ``score * fl32(1 / fl32(p))``, as
    torch computes it on a GPU, the reference's default device (config.py:63).
    """

    def __init__(self, device: torch.device, *, penalty_rounding: str = "division"):
        self.device = device
        if penalty_rounding not in _lib.PENALTY_ROUNDING:
            raise ValueError(f"penalty_rounding must be one of {sorted(_lib.PENALTY_ROUNDING)}")
        self.penalty_rounding = penalty_rounding
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
        B = len(sampling_params_list)
        N, V = logits.shape
        if sample_indices is None and B != N:
            raise ValueError(f"{B} sampling params for {N} logits rows")
        dev = logits.device
        slots = None
        if device_histories is not None:
            if history_requests is None or len(history_requests) != B:
                raise ValueError("history_requests must name one request per sampled row")
            slots = device_histories.slots(history_requests)
            if len(set(slots.tolist())) != B:
                raise ValueError("history_requests must name each request at most once")
            device_histories._check_room(slots)   # before any launch; counted once the append is issued
            max_hist = int(device_histories._len[slots].max()) if B else 0
            packed = PackedRows(sampling_params_list, None, V, slots=slots, slot_max_hist=max_hist,
                                penalty_rounding=self.penalty_rounding)
        else:
            packed = PackedRows(sampling_params_list, history_token_ids, V, penalty_rounding=self.penalty_rounding)
        d = packed.to_device(dev)
        if sample_indices is not None:
            sample_indices = sample_indices.to(device=dev, dtype=torch.int64)
            if sample_indices.numel() != B:
                raise ValueError("sample_indices must have one entry per sampling params")
        if uniforms is None:
            # rows whose request carries a seed draw a Philox uniform keyed by it and counted by
            # the history length (reproducible); the rest from ``generators`` or the device RNG
            seeded = [i for i, p in enumerate(sampling_params_list) if p.seed is not None]
            uniforms = self._draw_uniforms(B, dev, generators, skip=set(seeded))
            if seeded:
                if device_histories is not None:
                    steps = [int(device_histories._len[int(slots[i])]) for i in seeded]
                else:
                    steps = [len(history_token_ids[i]) if history_token_ids is not None and
                             history_token_ids[i] is not None else 0 for i in seeded]
                _lib.seeded_uniforms([sampling_params_list[i].seed for i in seeded], steps, seeded, uniforms)
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

    def _readback(self, out: torch.Tensor) -> SampledIds:
        """Copy ``out`` into a pinned host buffer behind an event on the current stream."""
        # one pinned buffer per call (torch's caching host allocator recycles them once
        # their handle is gone), so any number of calls may be in flight
        host = torch.empty(int(out.numel()), dtype=torch.int64, pin_memory=True)
        host.copy_(out, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(out.device))
        return SampledIds(out, host, ev)

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
