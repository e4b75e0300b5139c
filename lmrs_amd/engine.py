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

from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

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


class DecodeBatch:
    """Samples the next token of every live sequence with one launch."""

    def __init__(self, sequences: Sequence[SequenceState]):
        self.sequences = list(sequences)

    def live(self) -> List[int]:
        return [i for i, s in enumerate(self.sequences) if not s.finished]

    def step(self, logits) -> List[Optional[S.SampleOutput]]:
        """logits: [B, V] or [B, S, V] for the live sequences, in order.
        Returns one SampleOutput per sequence (None for finished ones)."""
        import torch

        rows = last_token_logits(logits)
        live = self.live()
        if rows.shape[0] != len(live):
            raise ValueError(f"{rows.shape[0]} logits rows for {len(live)} live sequences")
        if not live:
            return [None] * len(self.sequences)
        dev = rows.device
        seqs = [self.sequences[i] for i in live]
        uniforms, saved = [], []
        for s in seqs:
            saved.append(s.rng)
            u = 0.0
            if s.params.stochastic:
                u, s.rng = S.next_unit(s.rng)
            uniforms.append(u)
        off, ids = S.history_csr([s.generated for s in seqs], dev)
        res = S.sample_batch(rows.contiguous(), hist_offsets=off, hist_ids=ids,
                             temperature=[s.params.temperature for s in seqs],
                             top_k=[s.params.top_k for s in seqs], top_p=[s.params.top_p for s in seqs],
                             uniforms=uniforms)
        torch.cuda.current_stream(dev).synchronize()
        tok = res["token_ids"].cpu().numpy().view("uint32")
        lp = res["log_probs"].cpu().numpy()
        lg = res["logits"].cpu().numpy()
        st = res["status"].cpu().numpy() & 0xFF
        out: List[Optional[S.SampleOutput]] = [None] * len(self.sequences)
        for j, i in enumerate(live):
            s = self.sequences[i]
            if st[j] != S.ROW_OK:
                s.rng = saved[j]  # the reference draws only after validation
                raise S.SamplingError(f"sequence {i}: row status {int(st[j])}")
            o = S.SampleOutput(int(tok[j]), float(lp[j]), float(lg[j]))
            out[i] = o
            if s.eos_token is not None and o.token_id == s.eos_token:
                s.finished = True  # the EOS token is not appended (generation.rs:339-341)
            else:
                s.generated.append(o.token_id)
                if len(s.generated) >= s.config.max_tokens:
                    s.finished = True
        return out


def generate(model: Callable, prompts: Sequence[Sequence[int]], configs: Sequence[GenerationConfig],
             eos_token: Optional[int] = None, seeds: Optional[Sequence[int]] = None) -> List[List[int]]:
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
