"""The decode step of lmrs's engine over the batched HIP sampler.

The reference engine samples row by row: `Worker::run_batch` calls
`run_entry` for each batch entry, and each entry calls `Sampler::sample` on
its own row, with an empty history (crates/engine/src/worker/worker.rs:137-157).
`GenerationEngine::generate` loops the same way over one sequence, passing its
generated tokens as history (crates/engine/src/generation.rs:308-346).

Here one decode step is one `lmrs_sample_fwd` call over all live sequences,
and every row carries its own sequence's parameters, history and RNG state.
The per-row semantics are those of the reference's single-row calls:
- `sampler_for` maps a GenerationConfig to a strategy and a temperature
  (generation.rs:352-365);
- a sequence's RNG advances only when its strategy draws (strategies/mod.rs:44);
- a sequence stops on its EOS token or on reaching max_tokens, and the EOS token
  itself is not appended (generation.rs:339-341).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field
from collections.abc import Sequence as Seq
from typing import Callable, List, Optional

import numpy as np

from . import sampling as S


@dataclass(frozen=True)
class GenerationConfig:
    """GenerationConfig (crates/engine/src/generation.rs:71-98, default :121-130)."""

    max_tokens: int = 128
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: Optional[int] = None

    def __post_init__(self):
        # generation.rs:86-91 (a NaN temperature passes this check and fails in
        # Temperature::new when the sampler is built, as in the reference)
        if self.temperature <= 0.0:
            raise ValueError("temperature must be greater than zero")
        if not (0.0 <= self.top_p <= 1.0) or self.top_p == 0.0:
            raise ValueError("top_p must be in the range (0, 1]")


@dataclass(frozen=True)
class RowParams:
    """Kernel parameters of one row: what `sampler_for` builds, as numbers."""

    top_k: int
    top_p: float
    temperature: float
    stochastic: bool


def sampler_for(config: GenerationConfig) -> RowParams:
    """sampler_for (generation.rs:352-365): TopK when top_k is set, else TopP
    when top_p < 1, else Greedy; Temperature pushed when it is not 1."""
    if config.top_k is not None:
        strat = S.TopK(config.top_k)  # raises for 0, as TopK::new
    elif config.top_p < 1.0:
        strat = S.TopP(config.top_p)
    else:
        strat = S.Greedy()
    t = 1.0
    if config.temperature != 1.0:
        t = S.Temperature(config.temperature).value  # validates as Temperature::new
    return RowParams(strat.top_k, strat.top_p, t, strat.stochastic)


def last_token_logits(logits):
    """last_token_logits (crates/engine/src/worker/worker.rs:333-353) for a
    batch: [V] and [B, V] are taken as they are, [B, S, V] gives the last
    position of each sequence as [B, V]."""
    if logits.dim() == 1:
        return logits.reshape(1, -1)
    if logits.dim() == 2:
        return logits
    if logits.dim() == 3:
        if logits.shape[1] == 0:
            raise ValueError("cannot extract last token from empty sequence dim")
        return logits[:, -1, :]
    return logits.reshape(1, -1)


@dataclass
class SequenceState:
    """One sequence of a decode batch: its parameters, RNG state (the
    Sampler's LCG, seed 1 by default as SamplerConfig::new) and generated
    tokens (its sampling history)."""

    config: GenerationConfig
    eos_token: Optional[int] = None
    seed: int = 1
    generated: List[int] = field(default_factory=list)
    finished: bool = False

    def __post_init__(self):
        self.params = sampler_for(self.config)
        self.rng = max(int(self.seed), 1)


_ROW_MESSAGES = {S.ROW_EMPTY: "cannot sample from empty logits",
                 S.ROW_DISTRIBUTION: "logits produced an invalid probability distribution",
                 S.ROW_PARAM: "invalid sampling parameter", S.ROW_HISTORY: "history beyond the sampler's tables"}


class BatchSamplingError(S.SamplingError):
    """Some sequences of a decode step failed (SamplingError::Invalid per
    sequence); `errors` maps their indices to the reference's messages and
    `outputs` holds the step's outputs of the sequences that committed."""

    def __init__(self, errors: dict, outputs: list):
        super().__init__("; ".join(f"sequence {i}: {m}" for i, m in sorted(errors.items())))
        self.errors = errors
        self.outputs = outputs


class DecodeBatch:
    """Samples the next token of every live sequence with one launch.

    The live sequences' state stays on the device between steps: their
    histories in one [live, C] uint32 buffer (row j holds sequence j's
    generated tokens, then the padding id 0xFFFFFFFF, which is >= any vocab and
    so ignored by the sampler as repetition.rs:93 and presence.rs:113 ignore
    such ids), CSR offsets j * C, and the temperature / top-k / top-p arrays.
    A step copies the uniforms in, launches, copies the four outputs back in
    one transfer and appends the committed tokens in place; the buffers are
    rebuilt only when the live set changes or a history reaches C (doubled
    then)."""

    _PAD = 0xFFFFFFFF

    def __init__(self, sequences: Seq[SequenceState]):
        self.sequences = list(sequences)
        self._state_key = None
        self.timings: List[float] = []  # host wall time of each step (s), launch to outputs on the host

    def live(self) -> List[int]:
        return [i for i, s in enumerate(self.sequences) if not s.finished]

    def _device_state(self, live: List[int], dev):
        """(hist, offsets, temperature, top_k, top_p, outputs) for the live set,
        rebuilt when it or the capacity changed."""
        import torch

        need = max([len(self.sequences[i].generated) for i in live] + [1])
        key = (tuple(live), dev)
        if self._state_key == key and need < self._cap:
            return
        cap = 64
        while cap <= need:
            cap *= 2
        n = len(live)
        hist = torch.full((n, cap), -1, dtype=torch.int32, device=dev)  # -1 = 0xFFFFFFFF
        for j, i in enumerate(live):
            g = self.sequences[i].generated
            if g:
                hist[j, :len(g)] = torch.tensor([t if t < 2**31 else t - 2**32 for t in g], dtype=torch.int32)
        seqs = [self.sequences[i] for i in live]
        self._cap = cap
        self._hist = hist
        self._off = torch.arange(0, (n + 1) * cap, cap, dtype=torch.int64, device=dev)
        self._temp = torch.tensor([s.params.temperature for s in seqs], dtype=torch.float64, device=dev)
        self._topk = torch.tensor([s.params.top_k for s in seqs], dtype=torch.int32, device=dev)
        self._topp = torch.tensor([s.params.top_p for s in seqs], dtype=torch.float64, device=dev)
        # the four outputs as rows of one buffer: one copy back per step
        self._outbuf = torch.empty((4, n), dtype=torch.int32, device=dev)
        self._out = {"token_ids": self._outbuf[0], "log_probs": self._outbuf[1].view(torch.float32),
                     "logits": self._outbuf[2].view(torch.float32), "status": self._outbuf[3]}
        self._host = torch.empty((4, n), dtype=torch.int32, pin_memory=True)
        self._state_key = key

    def step(self, logits) -> List[Optional[S.SampleOutput]]:
        """logits: [B, V] or [B, S, V] for the live sequences, in order.
        Returns one SampleOutput per sequence (None for finished ones)."""
        import time

        import numpy as np
        import torch

        t0 = time.perf_counter()
        rows = last_token_logits(logits)
        live = self.live()
        if rows.shape[0] != len(live):
            raise ValueError(f"{rows.shape[0]} logits rows for {len(live)} live sequences")
        if not live:
            return [None] * len(self.sequences)
        dev = rows.device
        self._device_state(live, dev)
        seqs = [self.sequences[i] for i in live]
        uniforms, saved = [], []
        for s in seqs:
            saved.append(s.rng)
            u = 0.0
            if s.params.stochastic:
                u, s.rng = S.next_unit(s.rng)
            uniforms.append(u)
        stream = torch.cuda.current_stream(dev)
        S.sample_batch(rows.contiguous(), hist_offsets=self._off, hist_ids=self._hist,
                       temperature=self._temp, top_k=self._topk, top_p=self._topp,
                       uniforms=torch.tensor(uniforms, dtype=torch.float64).to(dev, non_blocking=True),
                       out=self._out, stream=stream)
        self._host.copy_(self._outbuf, non_blocking=True)
        stream.synchronize()
        h = self._host.numpy()
        tok = h[0].view(np.uint32)
        lp = h[1].view(np.float32)
        lg = h[2].view(np.float32)
        st = h[3] & 0xFF
        out: List[Optional[S.SampleOutput]] = [None] * len(self.sequences)
        # Every row's status is known before any state changes.  A failing
        # sequence keeps its generator as it was (the reference draws only
        # after validation, strategies/mod.rs:39-44) and gets no token; the
        # others commit, as each sequence's own generate loop would
        # (generation.rs:327-346), and the failures are raised together.
        errors = {}
        for j, i in enumerate(live):
            if st[j] != S.ROW_OK:
                self.sequences[i].rng = saved[j]
                errors[i] = _ROW_MESSAGES.get(int(st[j]), f"row status {int(st[j])}")
        app_rows, app_cols = [], []
        for j, i in enumerate(live):
            if i in errors:
                continue
            s = self.sequences[i]
            o = S.SampleOutput(int(tok[j]), float(lp[j]), float(lg[j]))
            out[i] = o
            if s.eos_token is not None and o.token_id == s.eos_token:
                s.finished = True  # the EOS token is not appended (generation.rs:339-341)
            else:
                app_rows.append(j)
                app_cols.append(len(s.generated))
                s.generated.append(o.token_id)
                if len(s.generated) >= s.config.max_tokens:
                    s.finished = True
        if app_rows:  # the committed tokens, appended on the device (where they already are)
            jr = torch.tensor(app_rows, dtype=torch.int64).to(dev, non_blocking=True)
            jc = torch.tensor(app_cols, dtype=torch.int64).to(dev, non_blocking=True)
            if max(app_cols) < self._cap:
                self._hist[jr, jc] = self._outbuf[0][jr]
            else:
                self._state_key = None  # a history reached the capacity: rebuilt next step
        self.timings.append(time.perf_counter() - t0)
        if errors:
            raise BatchSamplingError(errors, out)
        return out


def generate(model: Callable, prompts: Seq[Seq[int]], configs: Seq[GenerationConfig],
             eos_token: Optional[int] = None, seeds: Optional[Seq[int]] = None) -> List[List[int]]:
    """GenerationEngine::generate (generation.rs:308-346) for a batch of
    prompts: `model(step, tokens)` receives, for each live sequence in order,
    the tokens to run (the whole prompt at step 0, then its last token) and
    returns logits [B, S, V] or [B, V] on the GPU."""
    if any(len(p) == 0 for p in prompts):
        raise ValueError("prompt encoded to zero tokens")
    seqs = [SequenceState(c, eos_token, (seeds[i] if seeds else 1)) for i, c in enumerate(configs)]
    ctx = [list(p) for p in prompts]
    batch = DecodeBatch(seqs)
    for s in seqs:
        if s.config.max_tokens == 0:
            s.finished = True
    step = 0
    while batch.live():
        live = batch.live()
        tokens = [ctx[i] if step == 0 else [ctx[i][-1]] for i in live]
        out = batch.step(model(step, tokens))
        for i in live:
            o = out[i]
            if o is not None and not (eos_token is not None and o.token_id == eos_token):
                ctx[i].append(o.token_id)
        step += 1
        if step > max((c.max_tokens for c in configs), default=0) + 1:
            break
    return [s.generated for s in seqs]


# ---------------------------------------------------------------------------
# the wire format and the scheduler's side of a sample
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class GenerateParams:
    """GenerateParams (crates/server/src/types/openai.rs:101-158): the
    normalised request; temperature and top_p travel as f32 (defaults
    128 / 1.0 / 1.0 / None / no stop strings, :153-157)."""

    max_tokens: int = 128
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: Optional[int] = None
    stop: tuple = ()

    def __post_init__(self):
        object.__setattr__(self, "temperature", float(np.float32(self.temperature)))
        object.__setattr__(self, "top_p", float(np.float32(self.top_p)))

    @classmethod
    def from_request(cls, req: dict) -> "GenerateParams":
        """From a completion or chat request's optional fields (openai.rs:160-182)."""
        return cls(128 if req.get("max_tokens") is None else req["max_tokens"],  # unwrap_or(128): 0 stays 0
                   1.0 if req.get("temperature") is None else req["temperature"],
                   1.0 if req.get("top_p") is None else req["top_p"],
                   req.get("top_k"), tuple(req.get("stop") or ()))

    def to_generation_config(self) -> GenerationConfig:
        """ServerEngine::generate (crates/server/src/engine.rs:115-122): the f32
        values widened to f64, so T = 0.7 arrives as 0.699999988079071."""
        return GenerationConfig(self.max_tokens, float(self.temperature), float(self.top_p), self.top_k)


class FinishReason(enum.Enum):
    """FinishReason (crates/engine/src/sequence/status.rs:12-31)."""

    EOS = "eos"
    LENGTH = "length"
    STOPPED = "stopped"

    def __str__(self) -> str:
        return self.value


class SequenceStatus(enum.Enum):
    """SequenceStatus (status.rs:47-74)."""

    WAITING = "waiting"
    RUNNING = "running"
    SWAPPED = "swapped"
    FINISHED = "finished"
    ABORTED = "aborted"

    def can_prefill(self) -> bool:
        return self is SequenceStatus.WAITING

    def is_runnable(self) -> bool:
        return self in (SequenceStatus.WAITING, SequenceStatus.RUNNING)

    def is_terminal(self) -> bool:
        return self in (SequenceStatus.FINISHED, SequenceStatus.ABORTED)


class SequenceError(RuntimeError):
    """SequenceError (crates/engine/src/sequence/sequence.rs:8-27)."""


_TRANSITIONS = {
    (SequenceStatus.WAITING, SequenceStatus.RUNNING), (SequenceStatus.WAITING, SequenceStatus.FINISHED),
    (SequenceStatus.WAITING, SequenceStatus.ABORTED), (SequenceStatus.RUNNING, SequenceStatus.SWAPPED),
    (SequenceStatus.RUNNING, SequenceStatus.FINISHED), (SequenceStatus.RUNNING, SequenceStatus.ABORTED),
    (SequenceStatus.SWAPPED, SequenceStatus.RUNNING), (SequenceStatus.SWAPPED, SequenceStatus.ABORTED),
}


def validate_transition(src: SequenceStatus, dst: SequenceStatus) -> None:
    """validate_transition (status.rs:98-118)."""
    if src != dst and (src, dst) not in _TRANSITIONS:
        raise SequenceError(f"invalid sequence status transition from {src} to {dst}")


class Sequence:
    """Sequence (sequence.rs:48-213): the token buffer and lifecycle of one
    request, which receives each SampleOutput through append_sample."""

    def __init__(self, seq_id: int, prompt_tokens: Seq[int], max_new_tokens: int,
                 eos_token: Optional[int] = None):
        if len(prompt_tokens) == 0:
            raise SequenceError("sequence prompt cannot be empty")
        self.id = seq_id
        self.prompt_tokens = list(prompt_tokens)
        self.generated: List[S.SampleOutput] = []
        self.max_new_tokens = max_new_tokens
        self.eos_token = eos_token
        self.processed_len = 0
        self.status = SequenceStatus.WAITING
        self.finish_reason: Optional[FinishReason] = None

    def generated_token_ids(self) -> List[int]:
        return [o.token_id for o in self.generated]

    def total_len(self) -> int:
        return len(self.prompt_tokens) + len(self.generated)

    def pending_tokens(self) -> List[int]:
        return (self.prompt_tokens + self.generated_token_ids())[self.processed_len:self.total_len()]

    def has_pending_model_input(self) -> bool:
        return self.status.is_runnable() and self.processed_len < self.total_len()

    def _set_status(self, status: SequenceStatus) -> None:
        validate_transition(self.status, status)
        self.status = status

    def mark_processed(self, token_count: int) -> None:
        """sequence.rs:143-158."""
        processed = self.processed_len + token_count
        if processed > self.total_len():
            raise SequenceError(f"processed token count {processed} exceeds total token count {self.total_len()}")
        self.processed_len = processed
        if self.status is SequenceStatus.WAITING:
            self._set_status(SequenceStatus.RUNNING)

    def append_sample(self, sample: S.SampleOutput) -> None:
        """append_sample (sequence.rs:160-172): the sample is kept, EOS included;
        EOS finishes with Eos, reaching max_new_tokens with Length."""
        if self.status.is_terminal():
            raise SequenceError(f"sequence {self.id} is terminal")
        self.generated.append(sample)
        if self.eos_token is not None and sample.token_id == self.eos_token:
            self._finish(FinishReason.EOS)
        elif len(self.generated) >= self.max_new_tokens:
            self._finish(FinishReason.LENGTH)

    def stop(self) -> None:
        self._finish(FinishReason.STOPPED)

    def abort(self) -> None:
        self.finish_reason = None
        self._set_status(SequenceStatus.ABORTED)

    def swap_out(self) -> None:
        self._set_status(SequenceStatus.SWAPPED)

    def resume(self) -> None:
        self._set_status(SequenceStatus.RUNNING)

    def _finish(self, reason: FinishReason) -> None:
        self.finish_reason = reason
        self._set_status(SequenceStatus.FINISHED)


@dataclass(frozen=True)
class StepOutput:
    """StepOutput (crates/engine/src/executor/output.rs:16-44)."""

    sequence_id: int
    sample: S.SampleOutput


def run_batch(sampler: S.Sampler, logits, sequence_ids: Seq[int]) -> List[StepOutput]:
    """Worker::run_batch (crates/engine/src/worker/worker.rs:137-157) after the
    model: one launch samples the last-token logits of every entry with the
    worker's one Sampler and an empty history, as the reference's entry loop
    does, and pairs each sample with its sequence id."""
    rows = last_token_logits(logits)
    if rows.shape[0] != len(sequence_ids):
        raise ValueError(f"{rows.shape[0]} logits rows for {len(sequence_ids)} entries")
    if rows.shape[0] == 0:
        return []
    samples = sampler.sample_rows(rows.contiguous())
    return [StepOutput(i, o) for i, o in zip(sequence_ids, samples)]
