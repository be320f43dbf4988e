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
  draw.  When omitted they are drawn on the device from ``generators[i]``
  where given (the reference accepts ``generators`` but never uses them,
  sampler.py:26) and from the global CUDA generator otherwise.
* ``logits`` may be float32 or bfloat16 (bf16 is read directly; no
  ``.float()`` copy as at engine.py:236).

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
    """Per-row parameters and CSR histories packed for one ``ns_sample`` call."""

    def __init__(self, params: Sequence[SamplingParams], histories: Sequence, vocab: int):
        B = len(params)
        temp = np.empty(B, dtype=np.float32)
        topk = np.empty(B, dtype=np.int32)
        topp = np.empty(B, dtype=np.float32)
        pen = np.empty(B, dtype=np.float32)
        lens = np.zeros(B, dtype=np.int64)
        hist_rows = []
        for i, p in enumerate(params):
            t = float(p.temperature)
            # greedy rows are encoded as temperature 0 (sampler.py:47-50); others carry the
            # effective float32 temperature (sampler.py:41-46)
            temp[i] = 0.0 if t == 0.0 else np.float32(effective_temperature(t))
            k = int(p.top_k)
            topk[i] = min(max(k, -1), _I32_MAX)
            topp[i] = np.float32(float(p.top_p))
            rp = float(p.repetition_penalty)
            pen[i] = np.float32(rp)
            h = histories[i] if i < len(histories) else ()
            # only penalised rows index their history (sampler.py:33)
            if rp != 1.0 and len(h) > 0:
                a = np.asarray(h, dtype=np.int64)
                if a.size and (a.min() < 0 or a.max() >= vocab):
                    bad = int(a[(a < 0) | (a >= vocab)][0])
                    raise IndexError(f"history token id {bad} out of range for vocab {vocab} (row {i})")
                hist_rows.append(a.astype(np.int32))
                lens[i] = a.size
            else:
                hist_rows.append(None)
        self.batch = B
        self.row_kinds = _lib.row_kinds(temp, topk, vocab)
        self.temperature = temp
        self.top_k = topk
        self.top_p = topp
        self.penalty = pen
        self.max_hist = int(lens.max()) if B else 0
        if self.max_hist > _lib.NS_MAX_HISTORY:
            raise ValueError(f"history of {self.max_hist} tokens exceeds the supported {_lib.NS_MAX_HISTORY}")
        if self.max_hist > 0:
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
        buf = np.empty(4 * B + no + nh, dtype=np.int32)
        buf[0:B] = self.temperature.view(np.int32)
        buf[B:2 * B] = self.top_k
        buf[2 * B:3 * B] = self.top_p.view(np.int32)
        buf[3 * B:4 * B] = self.penalty.view(np.int32)
        if no:
            buf[4 * B:4 * B + no] = self.hist_offsets
            buf[4 * B + no:] = self.hist_ids
        host = torch.from_numpy(buf)
        if torch.device(device).type == "cuda":
            host = host.pin_memory()
        dev = host.to(device, non_blocking=True)
        out = {
            "temperature": dev[0:B].view(torch.float32),
            "top_k": dev[B:2 * B],
            "top_p": dev[2 * B:3 * B].view(torch.float32),
            "rep_penalty": dev[3 * B:4 * B].view(torch.float32),
            "hist_offsets": dev[4 * B:4 * B + no] if no else None,
            "hist_ids": dev[4 * B + no:] if no else None,
        }
        return out


class Sampler:
    """Drop-in for nanoserve.scheduler.sampler.Sampler (sampler.py:17-19)."""

    def __init__(self, device: torch.device):
        self.device = device
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
    ):
        """Sample one token per row; returns an int64 tensor on ``logits.device``.

        With ``return_probs=True`` returns ``(ids, probs)`` where ``probs`` holds the
        final (B, V) probabilities of every non-greedy row (sampler.py:76-80).
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
        packed = PackedRows(sampling_params_list, history_token_ids, V)
        d = packed.to_device(dev)
        if sample_indices is not None:
            sample_indices = sample_indices.to(device=dev, dtype=torch.int64)
            if sample_indices.numel() != B:
                raise ValueError("sample_indices must have one entry per sampling params")
        if uniforms is None:
            uniforms = self._draw_uniforms(B, dev, generators)
        else:
            uniforms = uniforms.to(device=dev, dtype=torch.float32).contiguous()
            if uniforms.numel() != B:
                raise ValueError("uniforms must have one entry per sampled row")
        out = torch.empty(B, dtype=torch.int64, device=dev)
        probs = torch.empty((B, V), dtype=torch.float32, device=dev) if return_probs else None
        if B > 0:
            _lib.sample_raw(logits, d["temperature"], d["top_k"], d["top_p"], d["rep_penalty"], uniforms, out,
                            sample_idx=sample_indices, hist_offsets=d["hist_offsets"], hist_ids=d["hist_ids"],
                            max_hist=packed.max_hist, out_probs=probs, row_kinds=packed.row_kinds)
        return (out, probs) if return_probs else out

    @staticmethod
    def _draw_uniforms(B: int, dev, generators) -> torch.Tensor:
        u = torch.rand(B, device=dev, dtype=torch.float32)
        if generators is not None:
            for i, g in enumerate(generators[:B]):
                if g is not None:
                    u[i] = torch.rand(1, generator=g, device=g.device, dtype=torch.float32).to(dev)[0]
        return u
