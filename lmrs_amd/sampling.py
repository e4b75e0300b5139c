"""Python binding of the HIP sampler's C-ABI (include/lmrs_sampling.h).

This is the host-side mirror of lmrs's ``crates/sampling`` API for Python
callers: ``Sampler`` / ``SamplerConfig`` / strategies / processors with the
reference's names and validation, plus ``sample_batch`` (per-row params in,
one token id per row out).  PyTorch only supplies device memory and the
stream; all sampling work runs in ``liblmrs_sampling.so``.  There is no CPU
fallback: importing this module without the built library raises.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblmrs_sampling.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "lmrs_sampling.h")

DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2

LMRS_OK = 0
ERR_NULL_ARGUMENT, ERR_BAD_DTYPE, ERR_BAD_SHAPE, ERR_LAUNCH, ERR_ALIGNMENT = -1, -2, -3, -4, -5
ROW_OK, ROW_EMPTY, ROW_DISTRIBUTION, ROW_PARAM, ROW_HISTORY = 0, 1, 2, 3, 4
ROW_NEAR_BOUNDARY = 0x100
GREEDY = -1  # top_k value selecting Greedy (greedy.rs:22-29); top_k = 1 is TopK(1)
MAX_VOCAB = 262144
MAX_HISTORY_DISTINCT = 12288  # distinct history tokens per row (LMRS_MAX_HISTORY_DISTINCT)
MAX_HISTORY_COUNT = 16383     # occurrences of one history token (LMRS_MAX_HISTORY_COUNT)


class SampleArgs(ctypes.Structure):
    """Mirror of ``lmrs_sample_args``."""

    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("vocab", ctypes.c_int64),
        ("row_stride", ctypes.c_int64),
        ("hist_offsets", ctypes.c_void_p),
        ("hist_ids", ctypes.c_void_p),
        ("repetition_penalty", ctypes.c_void_p),
        ("presence_penalty", ctypes.c_void_p),
        ("frequency_penalty", ctypes.c_void_p),
        ("temperature", ctypes.c_void_p),
        ("top_k", ctypes.c_void_p),
        ("top_p", ctypes.c_void_p),
        ("uniforms", ctypes.c_void_p),
        ("min_p", ctypes.c_void_p),
        ("token_ids", ctypes.c_void_p),
        ("log_probs", ctypes.c_void_p),
        ("logits_out", ctypes.c_void_p),
        ("status", ctypes.c_void_p),
        ("kept_count", ctypes.c_void_p),
        ("kept_mass", ctypes.c_void_p),
    ]


class LibraryMissing(RuntimeError):
    pass


_lib = None


def lib():
    """The loaded HIP library (raises LibraryMissing when it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(f"{LIB_PATH} is not built: run `python -m lmrs_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        L.lmrs_sample_fwd.argtypes = [ctypes.POINTER(SampleArgs), ctypes.c_void_p]
        L.lmrs_sample_fwd.restype = ctypes.c_int
        L.lmrs_process_logits_fwd.argtypes = [ctypes.POINTER(SampleArgs), ctypes.c_void_p, ctypes.c_void_p]
        L.lmrs_process_logits_fwd.restype = ctypes.c_int
        L.lmrs_sample_workspace_size.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int64]
        L.lmrs_sample_workspace_size.restype = ctypes.c_size_t
        L.lmrs_lm_head_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                       ctypes.c_void_p]
        L.lmrs_lm_head_fwd.restype = ctypes.c_int
        L.lmrs_sampling_version.argtypes = []
        L.lmrs_sampling_version.restype = ctypes.c_char_p
        _lib = L
    return _lib


class SamplingError(RuntimeError):
    """Mirror of SamplingError (crates/sampling/src/error.rs:20-39)."""


# ---------------------------------------------------------------------------
# device plumbing (torch tensors -> raw pointers)
# ---------------------------------------------------------------------------

def _torch():
    import torch  # noqa: WPS433 (imported lazily: only device plumbing)

    return torch


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _on_stream(stream, tensors) -> None:
    """Orders a launch on `stream` after the current stream's work (where the
    argument tensors were allocated and filled) and marks the tensors as used
    on `stream`, so that the caching allocator does not hand their memory to
    another allocation before `stream` has read them."""
    torch = _torch()
    cur = torch.cuda.current_stream(stream.device)
    if stream == cur:
        return
    stream.wait_stream(cur)
    for t in tensors:
        if t is not None:
            t.record_stream(stream)


def _dev_array(values, dtype, device):
    torch = _torch()
    if values is None:
        return None
    if isinstance(values, torch.Tensor):
        return values.to(device=device, dtype=dtype).contiguous()
    return torch.tensor(values, dtype=dtype, device=device)


def history_csr(histories: Sequence[Sequence[int]], device):
    """CSR (offsets int64 [B+1], ids uint32 as int32 storage) on `device`."""
    torch = _torch()
    offs = [0]
    flat: list[int] = []
    for h in histories:
        flat.extend(int(t) for t in h)
        offs.append(len(flat))
    off_t = torch.tensor(offs, dtype=torch.int64, device=device)
    ids = torch.tensor([t if t < 2**31 else t - 2**32 for t in flat] or [0], dtype=torch.int32, device=device)
    return off_t, ids


class PreparedBatch:
    """A sampling call with its argument block built once: ``launch`` only
    enqueues the kernels (for callers that repeat a step on fixed buffers)."""

    def __init__(self, args: SampleArgs, out: dict, keep: tuple):
        self.args = args
        self.out = out
        self._keep = keep

    def launch(self, stream) -> None:
        rc = lib().lmrs_sample_fwd(ctypes.byref(self.args), ctypes.c_void_p(stream.cuda_stream))
        if rc != LMRS_OK:
            raise SamplingError(f"lmrs_sample_fwd failed with code {rc}")


def prepare_batch(logits, *, hist_offsets=None, hist_ids=None, repetition_penalty=None,
                  presence_penalty=None, frequency_penalty=None, temperature=None, top_k=None,
                  top_p=None, uniforms=None, min_p=None, out=None, dist: bool = False) -> PreparedBatch:
    """Validates the host-side shapes and builds the argument block of
    ``lmrs_sample_fwd`` (per-row parameters as tensors or sequences of length
    B, None = neutral).  dist: also return each row's post-filter
    distribution size and mass (``kept_count``, ``kept_mass``)."""
    torch = _torch()
    if logits.dim() != 2:
        raise ValueError("logits must be [batch, vocab]")
    B, V = logits.shape
    if logits.stride(1) != 1 and V > 1:
        raise ValueError("logits rows must be contiguous")
    dev = logits.device
    dt = {torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32, torch.float16: DTYPE_F16}.get(logits.dtype)
    if dt is None:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    rp = _dev_array(repetition_penalty, torch.float32, dev)
    pp = _dev_array(presence_penalty, torch.float32, dev)
    fp = _dev_array(frequency_penalty, torch.float32, dev)
    tt = _dev_array(temperature, torch.float64, dev)
    tk = _dev_array(top_k, torch.int32, dev)
    tp = _dev_array(top_p, torch.float64, dev)
    uu = _dev_array(uniforms, torch.float64, dev)
    mp = _dev_array(min_p, torch.float64, dev)
    if out is None:
        out = {
            "token_ids": torch.empty(B, dtype=torch.int32, device=dev),
            "log_probs": torch.empty(B, dtype=torch.float32, device=dev),
            "logits": torch.empty(B, dtype=torch.float32, device=dev),
            "status": torch.empty(B, dtype=torch.int32, device=dev),
        }
    if dist and "kept_count" not in out:
        out["kept_count"] = torch.empty(B, dtype=torch.int32, device=dev)
        out["kept_mass"] = torch.empty(B, dtype=torch.float64, device=dev)
    args = SampleArgs(
        logits=_ptr(logits), dtype=dt, batch=B, vocab=V, row_stride=logits.stride(0) if B > 0 else V,
        hist_offsets=_ptr(hist_offsets), hist_ids=_ptr(hist_ids), repetition_penalty=_ptr(rp),
        presence_penalty=_ptr(pp), frequency_penalty=_ptr(fp), temperature=_ptr(tt), top_k=_ptr(tk),
        top_p=_ptr(tp), uniforms=_ptr(uu), min_p=_ptr(mp), token_ids=_ptr(out["token_ids"]),
        log_probs=_ptr(out["log_probs"]), logits_out=_ptr(out["logits"]), status=_ptr(out["status"]),
        kept_count=_ptr(out.get("kept_count")), kept_mass=_ptr(out.get("kept_mass")),
    )
    return PreparedBatch(args, out, (logits, rp, pp, fp, tt, tk, tp, uu, mp, hist_offsets, hist_ids))


def sample_batch(logits, *, hist_offsets=None, hist_ids=None, repetition_penalty=None,
                 presence_penalty=None, frequency_penalty=None, temperature=None, top_k=None,
                 top_p=None, uniforms=None, min_p=None, stream=None, out=None, dist: bool = False):
    """Samples one token per row of a [B, V] bf16/f32 CUDA tensor.

    Per-row parameters are tensors or sequences of length B (None = neutral;
    a negative min_p switches that row's min-p cut off).
    Returns dict(token_ids uint32-as-int32, log_probs f32, logits f32, status i32),
    all on the logits' device; the call is asynchronous on `stream`.
    """
    torch = _torch()
    pb = prepare_batch(logits, hist_offsets=hist_offsets, hist_ids=hist_ids,
                       repetition_penalty=repetition_penalty, presence_penalty=presence_penalty,
                       frequency_penalty=frequency_penalty, temperature=temperature, top_k=top_k,
                       top_p=top_p, uniforms=uniforms, min_p=min_p, out=out, dist=dist)
    s = stream if stream is not None else torch.cuda.current_stream(logits.device)
    _on_stream(s, list(pb._keep) + [v for k, v in pb.out.items() if k != "_keep"])
    pb.launch(s)
    out = pb.out
    # keep argument tensors alive until the stream has consumed them
    out["_keep"] = pb._keep
    return out


def process_logits(logits, *, hist_offsets=None, hist_ids=None, repetition_penalty=None,
                   presence_penalty=None, frequency_penalty=None, temperature=None, stream=None):
    """The processor chain only (LogitsProcessor::process, batched); returns [B, V] in the input dtype."""
    torch = _torch()
    dev = logits.device
    B, V = logits.shape
    dt = {torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}.get(logits.dtype)
    if dt is None:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    rp = _dev_array(repetition_penalty, torch.float32, dev)
    pp = _dev_array(presence_penalty, torch.float32, dev)
    fp = _dev_array(frequency_penalty, torch.float32, dev)
    tt = _dev_array(temperature, torch.float64, dev)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    out = torch.empty((B, V), dtype=logits.dtype, device=dev)
    args = SampleArgs(logits=_ptr(logits), dtype=dt, batch=B, vocab=V, row_stride=logits.stride(0) if B > 0 else V,
                      hist_offsets=_ptr(hist_offsets), hist_ids=_ptr(hist_ids), repetition_penalty=_ptr(rp),
                      presence_penalty=_ptr(pp), frequency_penalty=_ptr(fp), temperature=_ptr(tt),
                      status=_ptr(status))
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    _on_stream(s, [logits, rp, pp, fp, tt, hist_offsets, hist_ids, status, out])
    rc = lib().lmrs_process_logits_fwd(ctypes.byref(args), ctypes.c_void_p(out.data_ptr()),
                                       ctypes.c_void_p(s.cuda_stream))
    if rc != LMRS_OK:
        raise SamplingError(f"lmrs_process_logits_fwd failed with code {rc}")
    torch.cuda.current_stream(dev).synchronize() if stream is None else None
    return out, status


LM_HEAD_TILE = 64  # columns per tile_max entry of lmrs_lm_head_fwd


def lm_head(hidden, weight, *, tile_max: bool = True, stream=None):
    """LmHead::forward (crates/ops/src/embedding/lm_head.rs:33-35) on the matrix
    cores: logits [rows, V] bf16 = hidden [rows, H] bf16 @ weight[V, H]^T, and
    (tile_max) the sampling prologue of the epilogue, int64 [rows, ceil(V/64)]
    holding key << 32 | ~column of each 64-column tile's largest logit.
    Asynchronous on `stream` (default: the current stream)."""
    torch = _torch()
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [rows, H] and weight [V, H]")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("lm_head takes bf16 hidden states and weights")
    hidden, weight = hidden.contiguous(), weight.contiguous()
    rows, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    out = torch.empty((rows, V), dtype=torch.bfloat16, device=dev)
    tm = torch.empty((rows, (V + LM_HEAD_TILE - 1) // LM_HEAD_TILE), dtype=torch.int64, device=dev) if tile_max else None
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    _on_stream(s, [hidden, weight, out, tm])
    rc = lib().lmrs_lm_head_fwd(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(hidden.data_ptr()),
                                ctypes.c_void_p(weight.data_ptr()), rows, H, V, DTYPE_BF16,
                                ctypes.c_void_p(tm.data_ptr()) if tm is not None else None,
                                ctypes.c_void_p(s.cuda_stream))
    if rc != LMRS_OK:
        raise SamplingError(f"lmrs_lm_head_fwd failed with code {rc}")
    return out, tm


# ---------------------------------------------------------------------------
# mirror of the reference's single-row API (crates/sampling)
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class SampleOutput:
    """SampleOutput (crates/sampling/src/sampler/output.rs:14-44)."""

    token_id: int
    log_prob: float
    logit: float


class SamplingStrategy:
    """SamplingStrategy (strategies/mod.rs:16-19): maps onto kernel parameters."""

    top_k = 0
    top_p = 1.0
    min_p = -1.0  # off
    stochastic = True


class Greedy(SamplingStrategy):
    """Greedy (strategies/greedy.rs:19-29): sorted[0], no draw, no distribution check."""

    top_k = GREEDY
    stochastic = False


class BeamSearch(SamplingStrategy):
    """BeamSearch (strategies/beam.rs:23-50): the first sorted candidate, as Greedy."""

    top_k = GREEDY
    stochastic = False

    def __init__(self, width: int):
        if width == 0:
            raise SamplingError("beam width must be greater than zero")
        self.width = width


class TopK(SamplingStrategy):
    """TopK (strategies/top_k.rs:19-45)."""

    def __init__(self, k: int):
        if k <= 0:
            raise SamplingError("top_k must be greater than zero")
        self.k = k
        self.top_k = k


class TopP(SamplingStrategy):
    """TopP (strategies/top_p.rs:19-61)."""

    def __init__(self, p: float):
        if not math.isfinite(p) or p <= 0.0 or p > 1.0:
            raise SamplingError("top_p must be in (0, 1]")
        self.p = p
        self.top_p = p


class MinP(SamplingStrategy):
    """MinP (strategies/min_p.rs:19-55)."""

    def __init__(self, min_p: float):
        if not math.isfinite(min_p) or min_p < 0.0 or min_p > 1.0:
            raise SamplingError("min_p must be in [0, 1]")
        self.min_p = float(min_p)


class Temperature:
    """Temperature (logits/temperature.rs:24-72)."""

    def __init__(self, value: float):
        if not math.isfinite(value) or value <= 0.0:
            raise SamplingError("temperature must be finite and greater than zero")
        self.value = float(value)


class RepetitionPenalty:
    """RepetitionPenalty (logits/repetition.rs:38-117)."""

    def __init__(self, penalty: float):
        if not math.isfinite(penalty) or penalty <= 0.0:
            raise SamplingError("repetition penalty must be finite and greater than zero")
        self.penalty = float(penalty)


class FrequencyPresencePenalty:
    """FrequencyPresencePenalty (logits/presence.rs:41-130)."""

    def __init__(self, presence: float, frequency: float):
        if not math.isfinite(presence) or not math.isfinite(frequency):
            raise SamplingError("presence and frequency penalties must be finite")
        self.presence = float(presence)
        self.frequency = float(frequency)


def next_unit(state: int) -> tuple[float, int]:
    """The reference's LCG draw (strategies/mod.rs:57-61): returns (u, new_state)."""
    state = (state * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
    return ((state >> 11) & ((1 << 52) - 1)) / float(1 << 52), state


class SamplerConfig:
    """SamplerConfig (sampler/sampler.rs:21-72): strategy + LCG seed (default 1, min 1)."""

    def __init__(self, strategy: Optional[SamplingStrategy] = None):
        self.strategy = strategy if strategy is not None else Greedy()
        self.seed = 1

    def with_seed(self, seed: int) -> "SamplerConfig":
        self.seed = max(int(seed), 1)
        return self


class Sampler:
    """Sampler (sampler/sampler.rs:106-201) over the fused HIP kernel.

    Processors are applied in push order as the reference does, but only the
    reference's three processor kinds are supported, and each kind at most
    once, in the order Repetition -> Presence/Frequency -> Temperature (the
    fused kernel's fixed order); other orders raise SamplingError.
    """

    _ORDER = (RepetitionPenalty, FrequencyPresencePenalty, Temperature)

    def __init__(self, config: Optional[SamplerConfig] = None):
        config = config or SamplerConfig()
        self.strategy = config.strategy
        self.rng = config.seed
        self.processors: list = []

    def push_processor(self, processor) -> None:
        kinds = [type(p) for p in self.processors] + [type(processor)]
        pos = [self._ORDER.index(k) if k in self._ORDER else -1 for k in kinds]
        if -1 in pos or pos != sorted(set(pos)):
            raise SamplingError("the fused sampler applies Repetition, Presence/Frequency, Temperature in that order")
        self.processors.append(processor)

    def processor_count(self) -> int:
        return len(self.processors)

    def _processor_kw(self, rows: int) -> dict:
        kw = {}
        for p in self.processors:
            if isinstance(p, RepetitionPenalty):
                kw["repetition_penalty"] = [p.penalty] * rows
            elif isinstance(p, FrequencyPresencePenalty):
                kw["presence_penalty"] = [p.presence] * rows
                kw["frequency_penalty"] = [p.frequency] * rows
            elif isinstance(p, Temperature):
                kw["temperature"] = [p.value] * rows
        return kw

    def sample(self, logits, history: Sequence[int] = ()) -> SampleOutput:
        """One row (any shape, flattened), like Sampler::sample."""
        return self.sample_rows(logits.reshape(1, -1), [history])[0]

    def sample_rows(self, rows, histories: Optional[Sequence[Sequence[int]]] = None) -> list:
        """Sampler::sample on each row of a [B, V] tensor in order, as one
        launch: the rows share this sampler's processors and strategy, and
        the stochastic ones draw their uniforms from its one LCG in row order,
        as B successive calls would (the reference worker samples its batch
        entries this way, worker.rs:137-157).  On a failing row the error is
        raised and the LCG is left as the reference leaves it: advanced by the
        rows before it only, since a row draws after its validation
        (strategies/mod.rs:39-44)."""
        torch = _torch()
        B = rows.shape[0]
        hist = [list(h) for h in histories] if histories is not None else [[] for _ in range(B)]
        off, ids = history_csr(hist, rows.device)
        us, states = [], [self.rng]
        for _ in range(B):
            u = 0.0
            if self.strategy.stochastic:
                u, self.rng = next_unit(self.rng)
            us.append(u)
            states.append(self.rng)
        res = sample_batch(rows, hist_offsets=off, hist_ids=ids, top_k=[self.strategy.top_k] * B,
                           top_p=[self.strategy.top_p] * B, min_p=[self.strategy.min_p] * B, uniforms=us,
                           **self._processor_kw(B))
        torch.cuda.current_stream(rows.device).synchronize()
        st = res["status"].cpu().numpy() & 0xFF
        tok = res["token_ids"].cpu().numpy()
        lp = res["log_probs"].cpu().numpy()
        lg = res["logits"].cpu().numpy()
        out = []
        for j in range(B):
            if st[j] != ROW_OK:
                self.rng = states[j]
                raise SamplingError({ROW_EMPTY: "cannot sample from empty logits",
                                     ROW_DISTRIBUTION: "logits produced an invalid probability distribution",
                                     ROW_PARAM: "invalid sampling parameter",
                                     ROW_HISTORY: "history beyond the sampler's tables"}.get(int(st[j]), f"status {int(st[j])}"))
            out.append(SampleOutput(int(tok[j]) & 0xFFFFFFFF, float(lp[j]), float(lg[j])))
        return out
