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
  An implementation accurate to 1e-6 cuts somewhere inside it.  A row whose
  top-k survivors all hold one value has no zone: every implementation
  computes exp(0) = 1 for each and 1/n for each probability, so the arithmetic
  fixes the cut (two tied survivors at top_p = 0.5: the prefix 0.5 is not
  > 0.5, both are kept).
* the admissible cuts: every cut ``c`` in the zone (the last kept sorted
  position; ``c + 1`` tokens kept) is an alternative result of the row, with its
  own kept set, probabilities (``alternative()``) and allowed ids.  A row
  without a zone has one alternative, the oracle's own cut.  ``alt_kept[i]``
  lists the kept counts, ``alt_allowed[i]`` the allowed ids of each.
* allowed ids of one alternative: the kept tokens ``t`` with
  ``C[t-1] - 1e-6 <= u < C[t] + 1e-6`` (``C`` that alternative's float64
  cumulative mass in token-id order, ``C[-1] = 0``), plus its own pick.  For a
  row with no boundary within 1e-6 of ``u`` that is exactly the pick.
  ``allowed_ids[i]`` is their union over the row's alternatives: what an
  implementation may return when its kept count is not known.
* ``draw_boundary``: ``u`` lies within 1e-6 of the cumulative mass on either
  side of the picked token (the north-star exemption).
* ``topp_boundary``: the zone carries more than 1e-5 of mass.
* ``topp_tie_straddle``: tied values straddle the top-p cut.  The GPU path and
  this oracle agree there (lower id first), and so does ``torch.sort`` on the
  GPU, which the reference runs on (stable on ties, measured on ROCm torch).

The repetition penalty's division (sampler.py:37, ``score / p`` with ``p`` a
Python float) rounds differently by device: torch on the CPU divides
(correctly rounded), torch on a GPU multiplies by the reciprocal of the
Python float taken in float64 and rounded once (``x * fl32(1 / p)``, measured on
the MI355X).  ``penalty_rounding``
selects ``"division"`` (the default) or ``"reciprocal"``.

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
    zone_mass: np.ndarray         # (B,) float64 probability mass of sorted positions zone_lo+1 .. zone_hi
    zone_ids: list                # B arrays of token ids at sorted positions zone_lo+1 .. zone_hi
    nan_row: np.ndarray           # (B,) bool, probabilities replaced by 1/V (sampler.py:77-80)
    topp_boundary: np.ndarray     # (B,) bool, the zone carries more than 1e-5 of mass
    topp_tie_straddle: np.ndarray # (B,) bool
    draw_boundary: np.ndarray     # (B,) bool, u within 1e-6 of a cumulative mass next to the pick
    kept_mass: np.ndarray         # (B,) float64 top-p kept prefix mass (1 when top-p is off)
    allowed_ids: list             # B int64 arrays: the union of the alternatives' allowed ids
    alt_kept: list                # B int64 arrays: the kept count of each admissible top-p cut
    alt_allowed: list             # B lists of int64 arrays: the allowed ids of each alternative
    uniforms: np.ndarray          # (B,) float32 the draw's uniforms

    @property
    def exempt(self) -> np.ndarray:
        """Rows where more than one token id is allowed (never greedy rows)."""
        n = np.array([len(a) for a in self.allowed_ids], dtype=np.int64)
        return (n > 1) & ~self.greedy

    def alternative(self, i: int, n_kept: int):
        """(probabilities, allowed ids) of row ``i`` under the admissible cut keeping ``n_kept``
        tokens; ``None`` if ``n_kept`` is not one of ``alt_kept[i]``."""
        ks = self.alt_kept[i].tolist()
        if int(n_kept) not in ks:
            return None
        j = ks.index(int(n_kept))
        if int(n_kept) == int(self.n_kept[i]):
            return self.probs[i], self.alt_allowed[i][j]
        probs, allowed, _ = _cut_alternative(_topk_row(self.scaled[i], self.topk_thr[i]), int(n_kept) - 1,
                                             float(self.uniforms[i]))
        return probs, allowed


def effective_temperature(t: float) -> float:
    """sampler.py:42: ``max(t, 1e-6) if t > 0 else 1.0``."""
    return max(t, 1e-6) if t > 0 else 1.0


PENALTY_ROUNDINGS = ("division", "reciprocal")


def _apply_penalty(logits: torch.Tensor, penalties: Sequence[float], histories: Sequence,
                   penalty_rounding: str = "division") -> None:
    """sampler.py:31-38, in place on ``logits``.  ``"division"``: ``score / p`` correctly
    rounded, as torch computes it on the CPU; ``"reciprocal"``: ``score * fl32(1 / p)``, the
    float64 reciprocal of the Python float rounded once, as torch computes a tensor divided by
    a Python float on a GPU."""
    if penalty_rounding not in PENALTY_ROUNDINGS:
        raise ValueError(f"penalty_rounding must be one of {PENALTY_ROUNDINGS}")
    for i, p in enumerate(penalties):
        hist = histories[i]
        if p != 1.0 and len(hist) > 0:
            ids = torch.as_tensor(np.asarray(hist, dtype=np.int64))
            score = logits[i].index_select(0, ids)
            if penalty_rounding == "division":
                pos = score / p
            else:
                pos = score * float(np.float32(1.0 / p))
            score = torch.where(score < 0, score * p, pos)
            logits[i].index_copy_(0, ids, score)


def penalized_scaled(logits: torch.Tensor, temperature, penalties, histories, penalty_rounding="division"):
    """sampler.py:31-38 then :41-51 on a (B, V) float32 tensor (left unchanged): the logits
    after the repetition penalty, and after the penalty and the temperature division."""
    logits = logits.clone()
    _apply_penalty(logits, [float(p) for p in penalties], histories, penalty_rounding)
    penalized = logits.clone()
    temps = torch.tensor([effective_temperature(float(t)) for t in temperature], dtype=logits.dtype)
    return penalized, logits / temps.unsqueeze(1)


def _topk_row(scaled_row: torch.Tensor, thr) -> torch.Tensor:
    """sampler.py:58: the scaled row with the values below the top-k threshold removed."""
    if np.isnan(thr):
        return scaled_row.clone()
    t = torch.tensor(float(thr), dtype=scaled_row.dtype)
    return torch.where(scaled_row < t, torch.full_like(scaled_row, -float("inf")), scaled_row)


def _draw(probs_row: np.ndarray, u: float):
    """Inverse CDF (replacing sampler.py:87): the pick, the float64 CDF in token-id order."""
    V = probs_row.size
    cdf = probs_row.astype(np.float64).cumsum()
    j = int(np.searchsorted(cdf, u, side="right"))
    if j >= V:
        nz = np.flatnonzero(probs_row > 0)
        j = int(nz[-1]) if nz.size else V - 1
    return j, cdf


def _allowed(cdf: np.ndarray, kept: np.ndarray, u: float, pick: int) -> np.ndarray:
    """Kept tokens t with C[t-1] - 1e-6 <= u < C[t] + 1e-6 (C[-1] = 0), and the pick."""
    V = cdf.size
    a = int(np.searchsorted(cdf, u - BOUNDARY_EPS, side="right"))
    b = min(int(np.searchsorted(cdf, u + BOUNDARY_EPS, side="right")), V - 1)
    cand = np.flatnonzero(kept[a:b + 1]).astype(np.int64) + a if a <= b else np.zeros(0, dtype=np.int64)
    return np.union1d(cand, np.array([pick], dtype=np.int64)).astype(np.int64)


def _cut_alternative(topk_row: torch.Tensor, cut: int, u: float, sorted_idx=None):
    """Row after top-k, cut after sorted position ``cut`` (value descending, id ascending):
    its final probabilities, allowed ids and pick (sampler.py:64-80 with a given cut)."""
    if sorted_idx is None:
        _, sorted_idx = torch.sort(topk_row, descending=True, stable=True)
    masked = topk_row.clone()
    masked[sorted_idx[cut + 1:]] = -float("inf")
    probs = softmax_exact(masked)
    pnp = probs.numpy()
    pick, cdf = _draw(pnp, u)
    return probs, _allowed(cdf, np.isfinite(masked.numpy()), u, pick), pick


def sample(rows, temperature, top_k, top_p, repetition_penalty, histories, uniforms,
           penalty_rounding: str = "division") -> OracleResult:
    """Run the restated sampler on ``rows`` (B, V) float32 (numpy or CPU tensor)."""
    logits = torch.as_tensor(np.asarray(rows, dtype=np.float32)).clone()
    B, V = logits.shape
    temperature = [float(x) for x in temperature]
    top_k = [int(x) for x in top_k]
    top_p = [float(x) for x in top_p]
    penalties = [float(x) for x in repetition_penalty]
    u = np.asarray(uniforms, dtype=np.float32)

    penalized, logits = penalized_scaled(logits, temperature, penalties, histories, penalty_rounding)
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
    alt_cuts = [[] for _ in range(B)]     # (cut, allowed ids) of the admissible cuts but the oracle's own
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
            n_fin = int(torch.isfinite(sorted_logits).sum())
            # every survivor holds one value: probabilities 1/n in any arithmetic, no zone
            if n_fin > 0 and bool(sorted_logits[0] == sorted_logits[n_fin - 1]):
                lo = hi = J
            topp_cut[i], zone_lo[i], zone_hi[i] = J, lo, hi
            if not np.isnan(c64[-1]):
                # the cut lands in [lo, hi]: position lo is kept either way, so the
                # ambiguous tokens are the sorted positions lo+1 .. hi
                zone_mass[i] = c64[hi] - c64[lo]
                zone_ids[i] = sorted_idx[lo + 1:hi + 1].numpy().astype(np.int64)
                topp_boundary[i] = zone_mass[i] > ZONE_MASS_MAX
                kept_mass[i] = c64[J]
                ui = float(u[i])
                alt_cuts[i] = [(c, _cut_alternative(logits[i], c, ui, sorted_idx)[1])
                               for c in range(lo, min(hi, n_fin - 1) + 1) if c != J]
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
    n_kept = torch.isfinite(masked).sum(-1).numpy().astype(np.int64)
    ids = np.empty(B, dtype=np.int64)
    draw_boundary = np.zeros(B, dtype=bool)
    allowed = [np.zeros(0, dtype=np.int64) for _ in range(B)]
    alt_kept = [np.array([n_kept[i]], dtype=np.int64) for i in range(B)]
    alt_allowed = [[] for _ in range(B)]
    for i in range(B):
        if greedy[i]:
            ids[i] = int(argmax[i])
            allowed[i] = np.array([ids[i]], dtype=np.int64)
            alt_allowed[i] = [allowed[i]]
            continue
        ui = float(u[i])
        j, cdf = _draw(pnp[i], ui)
        ids[i] = j
        near = abs(cdf[j] - ui) < BOUNDARY_EPS
        if j > 0:
            near = near or abs(cdf[j - 1] - ui) < BOUNDARY_EPS
        draw_boundary[i] = near
        kept = np.ones(V, dtype=bool) if nan_np[i] else np.isfinite(masked[i].numpy())
        own = _allowed(cdf, kept, ui, j)
        counts, sets = [int(n_kept[i])], [own]
        for c, a_allowed in alt_cuts[i]:
            counts.append(c + 1)
            sets.append(a_allowed)
        order = np.argsort(counts, kind="stable")
        alt_kept[i] = np.asarray(counts, dtype=np.int64)[order]
        alt_allowed[i] = [sets[o] for o in order]
        allowed[i] = np.unique(np.concatenate(sets)).astype(np.int64)

    return OracleResult(ids=ids, probs=probs, penalized=penalized, scaled=scaled, masked=masked,
                        greedy=greedy, topk_thr=topk_thr, n_kept_topk=n_kept_topk, n_kept=n_kept,
                        topp_cut=topp_cut, zone_lo=zone_lo, zone_hi=zone_hi, zone_mass=zone_mass,
                        zone_ids=zone_ids, nan_row=nan_np, topp_boundary=topp_boundary,
                        topp_tie_straddle=tie_straddle, draw_boundary=draw_boundary,
                        kept_mass=kept_mass, allowed_ids=allowed, alt_kept=alt_kept, alt_allowed=alt_allowed,
                        uniforms=u.copy())


def sample_workload(w, rows_slice=None, penalty_rounding: str = "division") -> OracleResult:
    """Oracle over a ``workloads.Workload`` (optionally a slice of its rows)."""
    sl = rows_slice if rows_slice is not None else slice(None)
    return sample(w.rows[sl], w.temperature[sl], w.top_k[sl], w.top_p[sl], w.repetition_penalty[sl],
                  w.histories[sl], w.uniforms[sl], penalty_rounding=penalty_rounding)


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
