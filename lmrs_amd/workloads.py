"""Synthetic workloads C1..C5 (the benchmark configurations of the sampling path).

Each generator is deterministic in its seed and returns host (numpy) arrays:
logits [B, V] (uint16 bf16 bit patterns or float32), per-row parameters,
CSR history and the per-row uniforms.  Uniforms come from the reference's
own LCG (crates/sampling/src/strategies/mod.rs:57-61) seeded per row, so
the GPU and the CPU oracle consume identical draws.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

BASE_SEED = 20260501


def next_unit(state: int) -> tuple[float, int]:
    """One step of the reference LCG: returns (u in [0, 1), new state)."""
    state = (state * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
    return ((state >> 11) & ((1 << 52) - 1)) / float(1 << 52), state


def row_uniforms(batch: int, seed: int) -> np.ndarray:
    """u_r = next_unit(max(seed + r, 1)): one fresh sampler per row."""
    return np.array([next_unit(max(seed + r, 1))[0] for r in range(batch)], dtype=np.float64)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FFF
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


@dataclass
class Workload:
    name: str
    logits: np.ndarray            # [B, V] uint16 (bf16 bits) or float32
    repetition_penalty: np.ndarray
    presence_penalty: np.ndarray
    frequency_penalty: np.ndarray
    temperature: np.ndarray
    top_k: np.ndarray
    top_p: np.ndarray
    uniforms: np.ndarray
    hist_offsets: Optional[np.ndarray] = None  # int64 [B+1]
    hist_ids: Optional[np.ndarray] = None      # uint32
    notes: dict = field(default_factory=dict)
    min_p: Optional[np.ndarray] = None         # float64 [B]; None or negative = off

    @property
    def batch(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    @property
    def dtype(self) -> str:
        return "bf16" if self.logits.dtype == np.uint16 else "f32"

    @property
    def hist_len(self) -> int:
        if self.hist_offsets is None:
            return 0
        return int(np.max(np.diff(self.hist_offsets))) if self.batch else 0

    def algorithmic_bytes(self) -> int:
        """Bytes one step must move: logits once, history ids, per-row params and outputs."""
        esz = 2 if self.dtype == "bf16" else 4
        hist = 0 if self.hist_ids is None else int(self.hist_offsets[-1]) * 4
        mp = 0 if self.min_p is None else self.batch * 8
        return self.batch * self.vocab * esz + hist + self.batch * 44 + mp

    def rows(self, rows) -> "Workload":
        rows = np.asarray(rows)
        off = ids = None
        if self.hist_offsets is not None:
            parts = [self.hist_ids[self.hist_offsets[r]:self.hist_offsets[r + 1]] for r in rows]
            off = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.int64)
            ids = np.concatenate(parts).astype(np.uint32) if parts else np.zeros(0, np.uint32)
        return Workload(self.name, self.logits[rows], self.repetition_penalty[rows], self.presence_penalty[rows],
                        self.frequency_penalty[rows], self.temperature[rows], self.top_k[rows], self.top_p[rows],
                        self.uniforms[rows], off, ids, dict(self.notes),
                        None if self.min_p is None else self.min_p[rows])

    def truncated(self, vocab: int) -> "Workload":
        """The same rows cut to their first `vocab` logits (history ids beyond
        it stay: the sampler ignores ids >= vocab)."""
        if not 0 < vocab <= self.vocab:
            raise ValueError(f"vocab {vocab} outside 1..{self.vocab}")
        return Workload(self.name, np.ascontiguousarray(self.logits[:, :vocab]), self.repetition_penalty,
                        self.presence_penalty, self.frequency_penalty, self.temperature, self.top_k, self.top_p,
                        self.uniforms, self.hist_offsets, self.hist_ids, dict(self.notes, vocab=vocab), self.min_p)


def _params(B, rep=1.0, pres=0.0, freq=0.0, t=1.0, k=0, p=1.0):
    full = lambda v, dt: np.full(B, v, dtype=dt)  # noqa: E731
    return (full(rep, np.float32), full(pres, np.float32), full(freq, np.float32), full(t, np.float64),
            full(k, np.int32), full(p, np.float64))


def _zipf_history(rng, B, H, V, s=1.1):
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    perm = rng.permutation(V).astype(np.uint32)
    draws = np.searchsorted(cdf, rng.random((B, H)), side="left")
    ids = perm[np.minimum(draws, V - 1)].reshape(-1)
    off = np.arange(0, (B + 1) * H, H, dtype=np.int64)
    return off, ids.astype(np.uint32)


def c1(seed: int = BASE_SEED + 1, batch: int = 1) -> Workload:
    """Single-row CPU reference case: V=32000 f32 N(0,3^2) with 5 ids +8; T=0.8, k=50, p=0.9."""
    rng = np.random.default_rng(seed)
    V = 32000
    x = (rng.standard_normal((batch, V)) * 3.0).astype(np.float32)
    for r in range(batch):
        x[r, rng.choice(V, 5, replace=False)] += np.float32(8.0)
    rep, pres, freq, t, k, p = _params(batch, t=0.8, k=50, p=0.9)
    return Workload("C1", x, rep, pres, freq, t, k, p, row_uniforms(batch, seed))


def c2(seed: int = BASE_SEED + 2, batch: int = 64, vocab: int = 128256) -> Workload:
    """Heterogeneous batch: bf16 Student-t(3)*2.5; T~U[0.5,1.5], k in {0,1,20,50,1000}, p~U[0.8,1]."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_t(3, size=(batch, vocab)) * 2.5).astype(np.float32)
    rep, pres, freq, _, _, _ = _params(batch)
    t = rng.uniform(0.5, 1.5, batch).astype(np.float64)
    k = rng.choice(np.array([0, 1, 20, 50, 1000], dtype=np.int32), batch)
    p = rng.uniform(0.8, 1.0, batch).astype(np.float64)
    return Workload("C2", f32_to_bf16_bits(x), rep, pres, freq, t, k, p, row_uniforms(batch, seed))


def c3(seed: int = BASE_SEED + 3, batch: int = 256, vocab: int = 128256, hist: int = 2048) -> Workload:
    """Penalties + top-p: bf16 N(0,2.5^2), Zipf(1.1) history of 2048; rep 1.1, pres 0.5, freq 0.3, T=0.7, k=50, p=0.95."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((batch, vocab)) * 2.5).astype(np.float32)
    off, ids = _zipf_history(rng, batch, hist, vocab)
    rep, pres, freq, t, k, p = _params(batch, rep=1.1, pres=0.5, freq=0.3, t=0.7, k=50, p=0.95)
    return Workload("C3", f32_to_bf16_bits(x), rep, pres, freq, t, k, p, row_uniforms(batch, seed), off, ids)


def c4(seed: int = BASE_SEED + 4, batch: int = 1024, vocab: int = 151936, layout: str = "alternate") -> Workload:
    """Large batch: bf16 N(0,3^2); half Greedy (top_k = -1, the kernel's Greedy code), half full
    multinomial (k=0, p=1, T=1)."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((batch, vocab)) * 3.0).astype(np.float32)
    rep, pres, freq, t, k, p = _params(batch)
    greedy = (np.arange(batch) % 2 == 0) if layout == "alternate" else (np.arange(batch) < batch // 2)
    k[greedy] = -1  # Greedy
    return Workload("C4", f32_to_bf16_bits(x), rep, pres, freq, t, k, p, row_uniforms(batch, seed),
                    notes={"layout": layout})


def c5(seed: int = BASE_SEED + 5, batch: int = 512, vocab: int = 256000, hist: int = 512) -> Workload:
    """Top-p worst case: f32; half N(0,0.05^2), half N(0,1) with 3 ids +12; p=0.99, rep 1.05 over 512 uniform ids."""
    rng = np.random.default_rng(seed)
    x = np.empty((batch, vocab), dtype=np.float32)
    half = batch // 2
    x[:half] = (rng.standard_normal((half, vocab)) * 0.05).astype(np.float32)
    x[half:] = rng.standard_normal((batch - half, vocab)).astype(np.float32)
    for r in range(half, batch):
        x[r, rng.choice(vocab, 3, replace=False)] += np.float32(12.0)
    ids = rng.integers(0, vocab, size=batch * hist).astype(np.uint32)
    off = np.arange(0, (batch + 1) * hist, hist, dtype=np.int64)
    rep, pres, freq, t, k, p = _params(batch, rep=1.05, p=0.99)
    return Workload("C5", x, rep, pres, freq, t, k, p, row_uniforms(batch, seed), off, ids)


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5}
