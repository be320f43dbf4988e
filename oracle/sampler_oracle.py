"""CPU oracle: a restatement of NanoServe's ``Sampler.sample``.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product.

It follows nanoserve/scheduler/sampler.py:28-89 op by op with torch CPU ops at
float32 (the reference's arithmetic, ``requirements.txt:1`` pins torch), with the
reference's under-determined steps fixed the way the GPU path implements them:

* top-p (sampler.py:64) sorts with ``stable=True``: descending value, ascending
  token id on ties.  ``torch.sort(descending=True)`` is not stable on CPU.
* the cumulative sum of sorted probabilities (sampler.py:66) accumulates in
  float64 and rounds every prefix to float32, which is what CPU ``cumsum`` does
  for a float32 tensor; it is written out explicitly here.
* both softmaxes (sampler.py:65 and :76) are evaluated in float64 and rounded
  to float32.  The reference's float32 softmax rounding depends on the torch
  backend it runs on (CPU vectorised, CUDA, ROCm); all of them lie within
  1.6e-6 relative of this exactly-rounded value, which is what makes the top-p
  cut position reproducible to the 1e-6 zone described below.
* the ``torch.multinomial`` draw (sampler.py:87), which consumes the global RNG
  and cannot be replayed from per-row uniforms, is replaced by an inverse-CDF
  draw against one caller-supplied uniform ``u`` per row:
  ``token = min{i : C_i > u}`` where ``C`` is the float64 cumulative sum of the
  float32 probabilities in ascending token-id order; if rounding leaves no such
  ``i``, the last token with a non-zero probability.

Per row the oracle also reports what the parity tests need to compare an
implementation whose probabilities differ from these in the last ulps:

* the top-p *zone*: the sorted positions ``[zone_lo, zone_hi]`` whose float32
  prefix sum lies within 1e-6 of ``float32(top_p)`` (``zone_lo`` = first
  position with prefix > p - 1e-6, ``zone_hi`` = first with prefix > p + 1e-6).
  An implementation accurate to 1e-6 cuts somewhere inside it, so positions up
  to ``zone_lo`` are kept and positions after ``zone_hi`` removed by both;
  ``zone_ids`` lists the token ids at positions ``zone_lo+1 .. zone_hi`` (empty
  when the cut is unambiguous) and ``zone_mass`` their probability mass.
* ``topp_boundary``: the zone carries more than 1e-5 of mass (one heavy token
  sits on the cut), so the kept set itself is ambiguous.
* ``allowed_ids``: every token id an implementation may return for the row.
  An implementation whose kept set differs from this one only inside the zone
  renormalises by ``Q'`` instead of ``Q`` (kept masses, both at least
  ``Qmin``, the sorted prefix mass at ``zone_lo``), so each of its id-order
  cumulative masses lies within ``2 * zone_mass / Qmin`` of the oracle's
  (``zone_mass / Qmin`` from the rescaling of the kept tokens, as much again
  from the zone tokens themselves).  With ``draw_eps = 1e-6 + 2 * zone_mass /
  Qmin`` (just 1e-6 on rows without a zone), the allowed ids are the kept or
  zone tokens ``t`` with ``C[t-1] - draw_eps <= u < C[t] + draw_eps``, ``C``
  the oracle's float64 cumulative mass in token-id order.  For a row with no
  boundary within ``draw_eps`` of ``u`` that is exactly the oracle's pick.
* ``draw_boundary``: ``u`` lies within 1e-6 of the cumulative mass on either
  side of the picked token (the north-star exemption); ``draw_zone``: more
  than one id is allowed only because of the zone's widening.
* ``renorm``: ``zone_mass / Qmin``, the relative change of every kept
  probability an implementation may show on a row with a zone.
* ``topp_tie_straddle``: tied values straddle the top-p cut.  The GPU path and
  this oracle agree there (lower id first), and so does ``torch.sort`` on the
  GPU, which the reference runs on (stable on ties, measured on ROCm torch).

Pinned by tests/test_oracle_pins.py against closed forms (numpy float32
penalty and temperature, ``np.partition`` top-k, a numpy stable-argsort top-p,
float64 softmax), brute force on tiny vocabularies, invariants and a chi-square
test of the draw.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import numpy as np
import torch

BOUNDARY_EPS = 1e-6
ZONE_MASS_MAX = 1e-5


def softmax_exact(x: torch.Tensor) -> torch.Tensor:
    """float32 softmax evaluated in float64 and rounded (the oracle's softmax)."""
    return torch.softmax(x.double(), dim=-1).float()


@dataclass
class OracleResult:
    ids: np.ndarray               # (B,) int64 sampled token ids
    probs: torch.Tensor           # (B, V) float32 final probabilities (sampler.py:76-80)
    penalized: torch.Tensor       # (B, V) float32 after the repetition penalty (sampler.py:31-38)
    scaled: torch.Tensor          # (B, V) float32 after temperature (sampler.py:51)
    masked: torch.Tensor          # (B, V) float32 after top-k and top-p masking (sampler.py:53-73)
    greedy: np.ndarray            # (B,) bool, temperature == 0
    topk_thr: np.ndarray          # (B,) float32 k-th largest scaled logit, NaN when top-k is off
    n_kept_topk: np.ndarray       # (B,) int64 tokens surviving top-k (V when off)
    n_kept: np.ndarray            # (B,) int64 tokens with a finite masked logit after top-k and top-p
    topp_cut: np.ndarray          # (B,) int64 last kept position in the sorted order, -1 when top-p is off
    zone_lo: np.ndarray           # (B,) int64 first sorted position of the 1e-6 top-p zone (-1: off)
    zone_hi: np.ndarray           # (B,) int64 last sorted position of the zone
    zone_mass: np.ndarray         # (B,) float64 probability mass inside the zone
    zone_ids: list                # B arrays of token ids inside the zone
    nan_row: np.ndarray           # (B,) bool, probabilities replaced by 1/V (sampler.py:77-80)
    topp_boundary: np.ndarray     # (B,) bool
    topp_tie_straddle: np.ndarray # (B,) bool
    draw_boundary: np.ndarray     # (B,) bool, u within 1e-6 of a cumulative mass next to the pick
    draw_zone: np.ndarray         # (B,) bool, several ids allowed only through the zone's widening
    kept_mass: np.ndarray         # (B,) float64 top-p kept prefix mass (1 when top-p is off)
    renorm: np.ndarray            # (B,) float64 zone_mass / Qmin (0 without a zone)
    draw_eps: np.ndarray          # (B,) float64 the row's boundary band
    allowed_ids: list             # B int64 arrays: the ids an implementation may return

    @property
    def exempt(self) -> np.ndarray:
        """Rows where more than one token id is allowed (never greedy rows)."""
        n = np.array([len(a) for a in self.allowed_ids], dtype=np.int64)
        return (n > 1) & ~self.greedy


def effective_temperature(t: float) -> float:
    """sampler.py:42: ``max(t, 1e-6) if t > 0 else 1.0``."""
    return max(t, 1e-6) if t > 0 else 1.0


def _apply_penalty(logits: torch.Tensor, penalties: Sequence[float], histories: Sequence) -> None:
    """sampler.py:31-38, in place on ``logits``."""
    for i, p in enumerate(penalties):
        hist = histories[i]
        if p != 1.0 and len(hist) > 0:
            ids = torch.as_tensor(np.asarray(hist, dtype=np.int64))
            score = logits[i].index_select(0, ids)
            score = torch.where(score < 0, score * p, score / p)
            logits[i].index_copy_(0, ids, score)


def penalized_scaled(logits: torch.Tensor, temperature, penalties, histories):
    """sampler.py:31-38 then :41-51 on a (B, V) float32 tensor (left unchanged): the logits
    after the repetition penalty, and after the penalty and the temperature division."""
    logits = logits.clone()
    _apply_penalty(logits, [float(p) for p in penalties], histories)
    penalized = logits.clone()
    temps = torch.tensor([effective_temperature(float(t)) for t in temperature], dtype=logits.dtype)
    return penalized, logits / temps.unsqueeze(1)


def sample(rows, temperature, top_k, top_p, repetition_penalty, histories, uniforms) -> OracleResult:
    """Run the restated sampler on ``rows`` (B, V) float32 (numpy or CPU tensor)."""
    logits = torch.as_tensor(np.asarray(rows, dtype=np.float32)).clone()
    B, V = logits.shape
    temperature = [float(x) for x in temperature]
    top_k = [int(x) for x in top_k]
    top_p = [float(x) for x in top_p]
    penalties = [float(x) for x in repetition_penalty]
    u = np.asarray(uniforms, dtype=np.float32)

    penalized, logits = penalized_scaled(logits, temperature, penalties, histories)
    greedy = np.array([t == 0.0 for t in temperature], dtype=bool)
    scaled = logits.clone()

    # sampler.py:53-58
    topk_thr = np.full(B, np.nan, dtype=np.float32)
    n_kept_topk = np.full(B, V, dtype=np.int64)
    for i, k in enumerate(top_k):
        if k > 0 and k < V:
            vals, _ = torch.topk(logits[i], k)
            thr = vals[-1]
            logits[i] = torch.where(logits[i] < thr, torch.full_like(logits[i], -float("inf")), logits[i])
            topk_thr[i] = float(thr)
            n_kept_topk[i] = int((~(scaled[i] < thr)).sum())

    # sampler.py:60-73 with a stable sort and an explicit float64 accumulation
    topp_cut = np.full(B, -1, dtype=np.int64)
    zone_lo = np.full(B, -1, dtype=np.int64)
    zone_hi = np.full(B, -1, dtype=np.int64)
    zone_mass = np.zeros(B, dtype=np.float64)
    zone_ids = [np.zeros(0, dtype=np.int64) for _ in range(B)]
    topp_boundary = np.zeros(B, dtype=bool)
    tie_straddle = np.zeros(B, dtype=bool)
    kept_mass = np.ones(B, dtype=np.float64)
    qmin = np.ones(B, dtype=np.float64)
    for i, p in enumerate(top_p):
        if p < 1.0:
            sorted_logits, sorted_idx = torch.sort(logits[i], descending=True, stable=True)
            sorted_probs = softmax_exact(sorted_logits)
            cum_probs = sorted_probs.double().cumsum(-1).float()
            remove_sorted = cum_probs > p
            p32 = float(np.float32(p))
            c64 = cum_probs.double().numpy()

            def first_above(th):
                idx = np.flatnonzero(c64 > th)
                return int(idx[0]) if idx.size else V - 1

            J = first_above(p32)
            lo, hi = first_above(p32 - BOUNDARY_EPS), first_above(p32 + BOUNDARY_EPS)
            topp_cut[i], zone_lo[i], zone_hi[i] = J, lo, hi
            if not np.isnan(c64[-1]):
                # the cut lands in [lo, hi]: position lo is kept either way, so the
                # ambiguous tokens are the sorted positions lo+1 .. hi
                zone_mass[i] = c64[hi] - c64[lo]
                zone_ids[i] = sorted_idx[lo + 1:hi + 1].numpy().astype(np.int64)
                topp_boundary[i] = zone_mass[i] > ZONE_MASS_MAX
                kept_mass[i] = c64[J]
                qmin[i] = c64[lo]
            if J + 1 < V and bool(torch.isfinite(sorted_logits[J])):
                tie_straddle[i] = bool(sorted_logits[J + 1] == sorted_logits[J])
            remove_sorted[..., 1:] = remove_sorted[..., :-1].clone()
            remove_sorted[..., 0] = False
            remove_orig = torch.zeros_like(remove_sorted)
            remove_orig.scatter_(0, sorted_idx, remove_sorted)
            logits[i] = logits[i].masked_fill(remove_orig, -float("inf"))
    masked = logits.clone()

    # sampler.py:75-80
    probs = softmax_exact(logits)
    nan_rows = torch.isnan(probs).any(dim=-1)
    if nan_rows.any():
        probs[nan_rows] = 1.0 / V

    # sampler.py:82-83 (greedy) and the inverse-CDF draw replacing sampler.py:87
    argmax = torch.argmax(logits, dim=-1).numpy()
    pnp = probs.numpy()
    nan_np = nan_rows.numpy()
    ids = np.empty(B, dtype=np.int64)
    draw_boundary = np.zeros(B, dtype=bool)
    draw_zone = np.zeros(B, dtype=bool)
    renorm = np.zeros(B, dtype=np.float64)
    draw_eps = np.full(B, BOUNDARY_EPS, dtype=np.float64)
    allowed = [np.zeros(0, dtype=np.int64) for _ in range(B)]
    for i in range(B):
        if greedy[i]:
            ids[i] = int(argmax[i])
            allowed[i] = np.array([ids[i]], dtype=np.int64)
            continue
        cdf = pnp[i].astype(np.float64).cumsum()
        ui = float(u[i])
        j = int(np.searchsorted(cdf, ui, side="right"))
        if j >= V:
            nz = np.flatnonzero(pnp[i] > 0)
            j = int(nz[-1]) if nz.size else V - 1
        ids[i] = j
        near = abs(cdf[j] - ui) < BOUNDARY_EPS
        if j > 0:
            near = near or abs(cdf[j - 1] - ui) < BOUNDARY_EPS
        draw_boundary[i] = near
        if zone_mass[i] > 0.0:
            renorm[i] = zone_mass[i] / max(qmin[i], 1e-300)
            draw_eps[i] = BOUNDARY_EPS + 2.0 * renorm[i]
        eps = draw_eps[i]
        # kept or zone tokens t with C[t-1] - eps <= u < C[t] + eps (C[-1] = 0)
        a = int(np.searchsorted(cdf, ui - eps, side="right"))
        b = min(int(np.searchsorted(cdf, ui + eps, side="right")), V - 1)
        if a <= b:
            if nan_np[i]:
                cand = np.arange(a, b + 1, dtype=np.int64)
            else:
                keep = np.isfinite(masked[i, a:b + 1].numpy())
                cand = np.flatnonzero(keep).astype(np.int64) + a
                z = zone_ids[i]
                if len(z):
                    cand = np.union1d(cand, z[(z >= a) & (z <= b)])
        else:
            cand = np.zeros(0, dtype=np.int64)
        allowed[i] = np.union1d(cand, np.array([j], dtype=np.int64)).astype(np.int64)
        draw_zone[i] = len(allowed[i]) > 1 and not near

    n_kept = torch.isfinite(masked).sum(-1).numpy().astype(np.int64)
    return OracleResult(ids=ids, probs=probs, penalized=penalized, scaled=scaled, masked=masked,
                        greedy=greedy, topk_thr=topk_thr, n_kept_topk=n_kept_topk, n_kept=n_kept,
                        topp_cut=topp_cut, zone_lo=zone_lo, zone_hi=zone_hi, zone_mass=zone_mass,
                        zone_ids=zone_ids, nan_row=nan_np, topp_boundary=topp_boundary,
                        topp_tie_straddle=tie_straddle, draw_boundary=draw_boundary, draw_zone=draw_zone,
                        kept_mass=kept_mass, renorm=renorm, draw_eps=draw_eps, allowed_ids=allowed)


def sample_workload(w, rows_slice=None) -> OracleResult:
    """Oracle over a ``workloads.Workload`` (optionally a slice of its rows)."""
    sl = rows_slice if rows_slice is not None else slice(None)
    return sample(w.rows[sl], w.temperature[sl], w.top_k[sl], w.top_p[sl], w.repetition_penalty[sl],
                  w.histories[sl], w.uniforms[sl])


def reference_restatement_multinomial(logits: torch.Tensor, temperature, top_k, top_p, repetition_penalty,
                                      histories: List, generator=None) -> torch.Tensor:
    """The reference's own op sequence on CPU, multinomial draw included.

    This is sampler.py:28-89 restated without the parity fixes above (default
    unstable sort, ``torch.cumsum`` on float32, ``torch.multinomial``).  It is
    the timed CPU baseline; its ids are random and are not compared.
    """
    logits = logits.clone()
    num_seqs, vocab = logits.shape
    _apply_penalty(logits, [float(x) for x in repetition_penalty], histories)
    temps = torch.tensor([effective_temperature(float(t)) for t in temperature], dtype=logits.dtype)
    greedy = torch.tensor([float(t) == 0.0 for t in temperature])
    logits = logits / temps.unsqueeze(1)
    for i, k in enumerate(top_k):
        k = int(k)
        if k > 0 and k < vocab:
            topk_vals, _ = torch.topk(logits[i], k)
            threshold = topk_vals[-1]
            logits[i] = torch.where(logits[i] < threshold, torch.full_like(logits[i], -float("inf")), logits[i])
    for i, p in enumerate(top_p):
        p = float(p)
        if p < 1.0:
            sorted_logits, sorted_idx = torch.sort(logits[i], descending=True)
            sorted_probs = torch.softmax(sorted_logits, dim=-1)
            cum_probs = torch.cumsum(sorted_probs, dim=-1)
            remove_sorted = cum_probs > p
            remove_sorted[..., 1:] = remove_sorted[..., :-1].clone()
            remove_sorted[..., 0] = False
            remove_orig = torch.zeros_like(remove_sorted)
            remove_orig.scatter_(0, sorted_idx, remove_sorted)
            logits[i] = logits[i].masked_fill(remove_orig, -float("inf"))
    probs = torch.softmax(logits, dim=-1)
    nan_rows = torch.isnan(probs).any(dim=-1)
    if nan_rows.any():
        probs[nan_rows] = 1.0 / vocab
    argmax = torch.argmax(logits, dim=-1)
    sampled = torch.multinomial(probs, num_samples=1, generator=generator).squeeze(-1)
    return torch.where(greedy, argmax, sampled)
