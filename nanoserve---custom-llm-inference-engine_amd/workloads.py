"""Seeded synthetic sampler workloads (the five benchmark/parity configurations).

Every stream is drawn from ``numpy.random.SeedSequence(1000 + cfg).spawn(6)``
with one PCG64 generator per purpose (logits, boosts/prior, params, histories,
uniforms, sample positions), so the same arrays come out on any machine with
this numpy.  ``Workload.digest()`` hashes what was generated so a run can
confirm it regenerated identical inputs.

Configurations (vocab 128256 = Llama-3.2 unless stated):

  0  B=8, fp32 N(0, 2.5^2) + five tokens per row boosted by +8; t=0.8, k=50,
     p=0.9, penalty 1.1; histories of 64 uniform ids.
  1  B=64, logits as config 0; per-row t in {0, 0.7, 1.0, 1.3}, k in
     {0, 1, 20, 50, 1000}, p in {1.0, 0.95, 0.5}, penalty in {1.0, 1.2};
     histories of 512 Zipf(1.1) ids.
  2  B=256, N(0, 3^2) rounded to bf16 (stored bf16); t=1.0, k=50, p=0.95,
     penalty 1.1; histories of 2048 Zipf ids.  The headline configuration.
  3  B=128, vocab 256000, fp32 Gumbel(0,1) - 1.1*log(rank+1) with a per-row
     rank permutation; t=1.2, k off, p=0.99, no penalty.
  4  4096 x vocab fp32 N(0, 2.5^2) flat rows; 320 sampled rows (the last row of
     64 prefill chunks and 256 decodes, ascending as the scheduler builds them,
     nanoserve/scheduler/scheduler.py:240-246); params as config 1; histories
     of U[1, 4096] Zipf ids.

Penalty history ids are ``int32``; uniforms are float32 in [0, 1).
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

VOCAB_LLAMA32 = 128256
STREAMS = ("logits", "aux", "params", "hist", "uniform", "positions")


def _rngs(cfg: int):
    children = np.random.SeedSequence(1000 + cfg).spawn(len(STREAMS))
    return {name: np.random.Generator(np.random.PCG64(c)) for name, c in zip(STREAMS, children)}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even); returns uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    if not np.isfinite(x).all():
        raise ValueError("bf16 rounding helper expects finite values")
    bias = (u >> np.uint32(16)) & np.uint32(1)
    bias += np.uint32(0x7FFF)
    bias += u
    bias >>= np.uint32(16)
    return bias.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


_ZIPF_CDF = {}


def _zipf_cdf(vocab: int, s: float) -> np.ndarray:
    key = (vocab, s)
    if key not in _ZIPF_CDF:
        w = (np.arange(vocab, dtype=np.float64) + 1.0) ** (-s)
        cdf = np.cumsum(w)
        cdf /= cdf[-1]
        _ZIPF_CDF[key] = cdf
    return _ZIPF_CDF[key]


def zipf_ids(rng: np.random.Generator, n: int, vocab: int, perm: np.ndarray, s: float = 1.1) -> np.ndarray:
    """n ids from a bounded Zipf law over rank (P(r) ~ (r+1)^-s, r < vocab), mapped through perm."""
    cdf = _zipf_cdf(vocab, s)
    r = np.searchsorted(cdf, rng.random(n), side="right")
    r = np.minimum(r, vocab - 1)
    return perm[r].astype(np.int32)


@dataclass
class Workload:
    name: str
    vocab: int
    rows: np.ndarray                       # (B, V) float32 values of the sampled rows
    bf16_bits: Optional[np.ndarray]        # (B, V) uint16 when the logits are stored as bf16
    temperature: np.ndarray                # (B,) float64
    top_k: np.ndarray                      # (B,) int64
    top_p: np.ndarray                      # (B,) float64
    repetition_penalty: np.ndarray         # (B,) float64
    histories: List[np.ndarray]            # B arrays of int32 token ids
    uniforms: np.ndarray                   # (B,) float32 in [0, 1)
    n_rows_total: int = 0                  # rows of the flat logits tensor (== B unless sample_indices)
    sample_indices: Optional[np.ndarray] = None   # (B,) int64 ascending rows of the flat tensor
    filler_seed: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.rows.shape[0]

    @property
    def dtype(self) -> str:
        return "bf16" if self.bf16_bits is not None else "f32"

    def digest(self) -> str:
        h = hashlib.sha256()
        h.update(self.name.encode())
        h.update(np.ascontiguousarray(self.rows).tobytes())
        for a in (self.temperature, self.top_k, self.top_p, self.repetition_penalty, self.uniforms):
            h.update(np.ascontiguousarray(a).tobytes())
        for hist in self.histories:
            h.update(np.int64(len(hist)).tobytes())
            h.update(np.ascontiguousarray(hist, dtype=np.int32).tobytes())
        if self.sample_indices is not None:
            h.update(np.ascontiguousarray(self.sample_indices).tobytes())
        return h.hexdigest()

    def subset(self, n: int) -> "Workload":
        """The first n sampled rows (for quick runs); the flat layout is kept."""
        n = min(n, self.batch)
        return Workload(
            name=f"{self.name}[:{n}]", vocab=self.vocab, rows=self.rows[:n],
            bf16_bits=None if self.bf16_bits is None else self.bf16_bits[:n],
            temperature=self.temperature[:n], top_k=self.top_k[:n], top_p=self.top_p[:n],
            repetition_penalty=self.repetition_penalty[:n], histories=self.histories[:n],
            uniforms=self.uniforms[:n], n_rows_total=self.n_rows_total if self.sample_indices is not None else n,
            sample_indices=None if self.sample_indices is None else self.sample_indices[:n],
            filler_seed=self.filler_seed, notes=dict(self.notes))

    def device_logits(self, device, rotate: int = 0):
        """The flat logits tensor on ``device`` (bf16 or fp32 as the workload stores them).

        Non-sampled rows of a flat (chunked-prefill) layout are filled from a seeded
        torch generator; they are never read by the sampler.  ``rotate`` > 0 makes
        an independent copy with a different filler seed for buffer rotation.
        """
        import torch

        src = torch.from_numpy(self.bf16_bits.view(np.int16)).view(torch.bfloat16) if self.bf16_bits is not None \
            else torch.from_numpy(self.rows)
        if self.sample_indices is None:
            return src.to(device).contiguous()
        dt = src.dtype
        g = torch.Generator(device=device)
        g.manual_seed(self.filler_seed + rotate)
        out = torch.randn((self.n_rows_total, self.vocab), generator=g, device=device, dtype=torch.float32)
        out.mul_(2.5)
        out = out.to(dt)
        idx = torch.from_numpy(self.sample_indices).to(device)
        out.index_copy_(0, idx, src.to(device))
        return out


def _mixed_params(rng: np.random.Generator, B: int):
    t = rng.choice(np.array([0.0, 0.7, 1.0, 1.3]), size=B)
    k = rng.choice(np.array([0, 1, 20, 50, 1000], dtype=np.int64), size=B)
    p = rng.choice(np.array([1.0, 0.95, 0.5]), size=B)
    pen = rng.choice(np.array([1.0, 1.2]), size=B)
    return t, k, p, pen


def make_workload(cfg: int, batch: Optional[int] = None) -> Workload:
    """Build configuration ``cfg`` (0-4).  ``batch`` limits the sampled rows."""
    r = _rngs(cfg)
    V = 256000 if cfg == 3 else VOCAB_LLAMA32
    if cfg == 0:
        B = 8
    elif cfg == 1:
        B = 64
    elif cfg == 2:
        B = 256
    elif cfg == 3:
        B = 128
    elif cfg == 4:
        B = 320
    else:
        raise ValueError(f"unknown configuration {cfg}")
    n = B if batch is None else min(batch, B)
    bf16 = None
    n_total = n
    sample_idx = None
    notes = {}

    # ---- logits of the sampled rows
    if cfg in (0, 1):
        rows = r["logits"].normal(0.0, 2.5, size=(B, V)).astype(np.float32)[:n]
        for i in range(n):
            pos = r["aux"].choice(V, size=5, replace=False)
            rows[i, pos] += np.float32(8.0)
    elif cfg == 2:
        raw = r["logits"].normal(0.0, 3.0, size=(n, V)).astype(np.float32)
        bf16 = f32_to_bf16_bits(raw)
        rows = bf16_bits_to_f32(bf16)
    elif cfg == 3:
        rows = np.empty((n, V), dtype=np.float32)
        prior = (-1.1 * np.log(np.arange(V, dtype=np.float64) + 1.0))
        for i in range(n):
            perm = r["aux"].permutation(V)
            g = r["logits"].gumbel(0.0, 1.0, size=V)
            rows[i] = (g + prior[perm]).astype(np.float32)
    else:  # cfg == 4
        rows = r["logits"].normal(0.0, 2.5, size=(n, V)).astype(np.float32)

    # ---- per-row params
    if cfg == 0:
        t = np.full(n, 0.8); k = np.full(n, 50, dtype=np.int64); p = np.full(n, 0.9); pen = np.full(n, 1.1)
    elif cfg in (1, 4):
        t, k, p, pen = _mixed_params(r["params"], B)
        t, k, p, pen = t[:n], k[:n], p[:n], pen[:n]
    elif cfg == 2:
        t = np.full(n, 1.0); k = np.full(n, 50, dtype=np.int64); p = np.full(n, 0.95); pen = np.full(n, 1.1)
    else:
        t = np.full(n, 1.2); k = np.full(n, -1, dtype=np.int64); p = np.full(n, 0.99); pen = np.full(n, 1.0)

    # ---- histories
    hr = r["hist"]
    perm = hr.permutation(V)
    if cfg == 0:
        hists = [hr.integers(0, V, size=64).astype(np.int32) for _ in range(B)][:n]
    elif cfg == 1:
        hists = [zipf_ids(hr, 512, V, perm) for _ in range(B)][:n]
    elif cfg == 2:
        hists = [zipf_ids(hr, 2048, V, perm) for _ in range(B)][:n]
    elif cfg == 3:
        hists = [np.zeros(0, dtype=np.int32) for _ in range(n)]
    else:
        lens = hr.integers(1, 4097, size=B)
        hists = [zipf_ids(hr, int(L), V, perm) for L in lens][:n]

    u = r["uniform"].random(B, dtype=np.float32)[:n]

    if cfg == 4:
        # flat layout: 256 decode rows (q_len 1) and 64 prefill chunks (q_len 1..512, sum 3840),
        # interleaved in a seeded order; the sampled row of each sequence is its last one.
        pr = r["positions"]
        cuts = np.sort(pr.choice(np.arange(1, 3840), size=63, replace=False))
        chunk_lens = np.diff(np.concatenate([[0], cuts, [3840]]))
        # keep every chunk within 1..512 by repeatedly splitting the mass of oversize chunks
        while chunk_lens.max() > 512:
            big = int(np.argmax(chunk_lens)); small = int(np.argmin(chunk_lens))
            move = chunk_lens[big] - 512
            chunk_lens[big] -= move
            chunk_lens[small] += move
        qlens = np.concatenate([np.ones(256, dtype=np.int64), chunk_lens.astype(np.int64)])
        order = pr.permutation(len(qlens))
        qlens = qlens[order]
        ends = np.cumsum(qlens) - 1
        assert ends[-1] == 4095
        sample_idx = ends.astype(np.int64)[:n]
        n_total = 4096
        notes["query_lens"] = qlens

    return Workload(name=f"c{cfg}", vocab=V, rows=rows, bf16_bits=bf16, temperature=np.asarray(t, np.float64),
                    top_k=np.asarray(k, np.int64), top_p=np.asarray(p, np.float64),
                    repetition_penalty=np.asarray(pen, np.float64), histories=list(hists), uniforms=u,
                    n_rows_total=n_total, sample_indices=sample_idx, filler_seed=77_000 + cfg, notes=notes)


def make_mixed_decode(batch: int = 256, seed: int = 1005) -> Workload:
    """A decode batch of bf16 rows (N(0, 3^2) rounded to bf16, vocab 128256) with the
    mixed per-row parameters of configuration 1 (greedy, top-k off and k > 64 among
    them) and 512 Zipf history ids per row: a batch large enough for the
    one-workgroup-per-row launch that still holds rows with top-k off or k > 64."""
    children = np.random.SeedSequence(seed).spawn(len(STREAMS))
    r = {name: np.random.Generator(np.random.PCG64(c)) for name, c in zip(STREAMS, children)}
    V = VOCAB_LLAMA32
    raw = r["logits"].normal(0.0, 3.0, size=(batch, V)).astype(np.float32)
    bf16 = f32_to_bf16_bits(raw)
    rows = bf16_bits_to_f32(bf16)
    t, k, p, pen = _mixed_params(r["params"], batch)
    perm = r["hist"].permutation(V)
    hists = [zipf_ids(r["hist"], 512, V, perm) for _ in range(batch)]
    u = r["uniform"].random(batch, dtype=np.float32)
    return Workload(name=f"mixed-bf16-b{batch}", vocab=V, rows=rows, bf16_bits=bf16,
                    temperature=np.asarray(t, np.float64), top_k=np.asarray(k, np.int64),
                    top_p=np.asarray(p, np.float64), repetition_penalty=np.asarray(pen, np.float64),
                    histories=hists, uniforms=u, n_rows_total=batch)


def algorithmic_bytes(w: Workload) -> int:
    """Compulsory HBM bytes of one sampler call over ``w``.

    Per sampled row: V * s_in (the logits row) + 4 * H for penalized rows with a
    history + 32 (f32 temperature, i32 top_k, f32 top_p, f32 penalty, f32
    uniform, i32 CSR offset, i64 output id) + 8 when sample indices are given.
    """
    s_in = 2 if w.bf16_bits is not None else 4
    total = 0
    for i in range(w.batch):
        b = w.vocab * s_in + 32
        if w.repetition_penalty[i] != 1.0 and len(w.histories[i]) > 0:
            b += 4 * len(w.histories[i])
        if w.sample_indices is not None:
            b += 8
        total += b
    return total
