"""ctypes view of the CPU oracle (oracle/liblmrs_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
as the checker, and by ``bench.py``'s ``cpu_baseline`` leg.  The product path
(``lmrs_amd``) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblmrs_oracle.so")

OK, ERR_EMPTY, ERR_DISTRIBUTION, ERR_PARAM = 0, 1, 2, 3
GREEDY = -1  # top_k value that selects Greedy (greedy.rs:22-29); top_k = 1 is TopK(1)


class Output(ctypes.Structure):
    _fields_ = [("token_id", ctypes.c_uint32), ("log_prob", ctypes.c_float), ("logit", ctypes.c_float)]


class Params(ctypes.Structure):
    _fields_ = [
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("temperature", ctypes.c_double),
        ("top_k", ctypes.c_int64),
        ("top_p", ctypes.c_double),
        ("min_p", ctypes.c_double),
    ]


class Diag(ctypes.Structure):
    _fields_ = [
        ("cdf_margin", ctypes.c_double),
        ("top_p_margin", ctypes.c_double),
        ("min_p_margin", ctypes.c_double),
        ("cum_before", ctypes.c_double),
        ("sum_kept", ctypes.c_double),
        ("weight", ctypes.c_double),
        ("n_candidates", ctypes.c_int64),
        ("n_kept", ctypes.c_int64),
    ]


def build() -> None:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, i64, f64, f32, u64p = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)
        L.lmrs_oracle_bf16_from_f32_host.argtypes = [f32]
        L.lmrs_oracle_bf16_from_f32_host.restype = ctypes.c_uint16
        L.lmrs_oracle_bf16_from_f32_dev.argtypes = [f32]
        L.lmrs_oracle_bf16_from_f32_dev.restype = ctypes.c_uint16
        L.lmrs_oracle_f32_from_bf16.argtypes = [ctypes.c_uint16]
        L.lmrs_oracle_f32_from_bf16.restype = f32
        L.lmrs_oracle_next_unit.argtypes = [u64p]
        L.lmrs_oracle_next_unit.restype = f64
        L.lmrs_oracle_total_cmp.argtypes = [f32, f32]
        L.lmrs_oracle_total_cmp.restype = ctypes.c_int
        L.lmrs_oracle_sorted_indices.argtypes = [P, i64, P]
        L.lmrs_oracle_sorted_indices.restype = None
        outp = ctypes.POINTER(Output)
        L.lmrs_oracle_greedy.argtypes = [P, i64, outp]
        L.lmrs_oracle_beam.argtypes = [P, i64, i64, outp]
        L.lmrs_oracle_top_k.argtypes = [P, i64, i64, u64p, outp]
        L.lmrs_oracle_top_p.argtypes = [P, i64, f64, u64p, outp]
        L.lmrs_oracle_min_p.argtypes = [P, i64, f64, u64p, outp]
        L.lmrs_oracle_repetition.argtypes = [P, ctypes.c_int, i64, f32, P, i64]
        L.lmrs_oracle_presence.argtypes = [P, ctypes.c_int, i64, f32, f32, P, i64]
        L.lmrs_oracle_temperature.argtypes = [P, ctypes.c_int, i64, f64]
        L.lmrs_oracle_sample_row.argtypes = [P, ctypes.c_int, i64, P, i64, ctypes.POINTER(Params), f64,
                                             outp, ctypes.POINTER(Diag), P]
        L.lmrs_oracle_sample_batch.argtypes = [P, ctypes.c_int, i64, i64, i64, P, P, P, P, P, P, P,
                                               ctypes.c_int]
        L.lmrs_oracle_linear_bf16.argtypes = [P, P, i64, i64, i64, P, P, P]
        L.lmrs_oracle_linear_bf16.restype = None
        _lib = L
    return _lib


def linear_bf16(x_bits: np.ndarray, w_bits: np.ndarray):
    """linear_kernel (tensor_ffi.cu:230-258) for bf16 without bias: returns
    (y bf16 bits [rows, out], f32 sums [rows, out], sum |x w| [rows, out])."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, n_in = x.shape
    n_out = w.shape[0]
    assert w.shape[1] == n_in
    y = np.empty((rows, n_out), dtype=np.uint16)
    acc = np.empty((rows, n_out), dtype=np.float32)
    sa = np.empty((rows, n_out), dtype=np.float64)
    lib().lmrs_oracle_linear_bf16(_ptr(x), _ptr(w), rows, n_in, n_out, _ptr(y), _ptr(acc), _ptr(sa))
    return y, acc, sa


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


# ---- scalar helpers --------------------------------------------------------

def bf16_host(x: float) -> int:
    return lib().lmrs_oracle_bf16_from_f32_host(float(x))


def bf16_dev(x: float) -> int:
    return lib().lmrs_oracle_bf16_from_f32_dev(float(x))


def f32_from_bf16(b: int) -> float:
    return lib().lmrs_oracle_f32_from_bf16(int(b))


def next_unit(state: int) -> tuple[float, int]:
    s = ctypes.c_uint64(state)
    u = lib().lmrs_oracle_next_unit(ctypes.byref(s))
    return u, s.value


def total_cmp(a: float, b: float) -> int:
    return lib().lmrs_oracle_total_cmp(a, b)


def sorted_indices(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    order = np.empty(len(x), dtype=np.int64)
    lib().lmrs_oracle_sorted_indices(_ptr(x), len(x), _ptr(order))
    return order


# ---- strategies -----------------------------------------------------------

def _strategy(fn, x, *args, rng=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = Output()
    if rng is None:
        st = fn(_ptr(x), len(x), *args, ctypes.byref(out))
        return st, (out.token_id, out.log_prob, out.logit)
    s = ctypes.c_uint64(rng)
    st = fn(_ptr(x), len(x), *args, ctypes.byref(s), ctypes.byref(out))
    return st, (out.token_id, out.log_prob, out.logit), s.value


def greedy(x):
    return _strategy(lib().lmrs_oracle_greedy, x)


def beam(x, width):
    return _strategy(lib().lmrs_oracle_beam, x, int(width))


def top_k(x, k, rng):
    return _strategy(lib().lmrs_oracle_top_k, x, int(k), rng=rng)


def top_p(x, p, rng):
    return _strategy(lib().lmrs_oracle_top_p, x, float(p), rng=rng)


def min_p(x, p, rng):
    return _strategy(lib().lmrs_oracle_min_p, x, float(p), rng=rng)


# ---- processors (numpy rows; bf16 rows are uint16 bit patterns) -----------

def _proc_row(x):
    x = np.array(x, copy=True)
    if x.dtype == np.uint16:
        return x, 0
    return np.ascontiguousarray(x, dtype=np.float32), 2


def _hist(h):
    return np.ascontiguousarray(np.asarray(h, dtype=np.uint32).reshape(-1))


def repetition(x, penalty, history):
    row, dt = _proc_row(x)
    h = _hist(history)
    st = lib().lmrs_oracle_repetition(_ptr(row), dt, len(row), float(penalty), _ptr(h), len(h))
    return st, row


def presence(x, presence_, frequency, history):
    row, dt = _proc_row(x)
    h = _hist(history)
    st = lib().lmrs_oracle_presence(_ptr(row), dt, len(row), float(presence_), float(frequency), _ptr(h), len(h))
    return st, row


def temperature(x, t):
    row, dt = _proc_row(x)
    st = lib().lmrs_oracle_temperature(_ptr(row), dt, len(row), float(t))
    return st, row


# ---- composed sampler -----------------------------------------------------

def make_params(repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0,
                temperature=1.0, top_k=0, top_p=1.0, min_p=-1.0) -> Params:
    return Params(repetition_penalty, presence_penalty, frequency_penalty, temperature, int(top_k), top_p, min_p)


def sample_row(logits, history, params: Params, u: float, want_processed=False):
    """One row; logits uint16 (bf16 bits) or float32. Returns (status, (id, logprob, logit), diag, processed)."""
    row, dt = _proc_row(logits)
    h = _hist(history) if history is not None else np.zeros(0, np.uint32)
    out, diag = Output(), Diag()
    proc = np.empty(len(row), np.float32) if want_processed else None
    st = lib().lmrs_oracle_sample_row(_ptr(row), dt, len(row), _ptr(h), len(h), ctypes.byref(params), float(u),
                                      ctypes.byref(out), ctypes.byref(diag), _ptr(proc))
    return st, (out.token_id, out.log_prob, out.logit), diag, proc


def sample_batch(logits: np.ndarray, hist_offsets, hist_ids, params_list, uniforms, n_threads=1):
    """logits: [B, V] uint16 or float32.  Returns dict of numpy arrays."""
    logits = np.ascontiguousarray(logits)
    dt = 0 if logits.dtype == np.uint16 else 2
    B, V = logits.shape
    P = (Params * B)(*params_list)
    u = np.ascontiguousarray(uniforms, dtype=np.float64)
    off = None if hist_offsets is None else np.ascontiguousarray(hist_offsets, dtype=np.int64)
    ids = None if hist_ids is None else np.ascontiguousarray(hist_ids, dtype=np.uint32)
    outs = (Output * B)()
    diags = (Diag * B)()
    status = np.zeros(B, np.int32)
    lib().lmrs_oracle_sample_batch(_ptr(logits), dt, B, V, V, _ptr(off), _ptr(ids), ctypes.cast(P, ctypes.c_void_p),
                                   _ptr(u), ctypes.cast(outs, ctypes.c_void_p), ctypes.cast(diags, ctypes.c_void_p),
                                   _ptr(status), int(n_threads))
    return {
        "status": status,
        "token_id": np.array([o.token_id for o in outs], np.uint32),
        "log_prob": np.array([o.log_prob for o in outs], np.float32),
        "logit": np.array([o.logit for o in outs], np.float32),
        "cdf_margin": np.array([d.cdf_margin for d in diags]),
        "top_p_margin": np.array([d.top_p_margin for d in diags]),
        "min_p_margin": np.array([d.min_p_margin for d in diags]),
        "n_candidates": np.array([d.n_candidates for d in diags]),
        "n_kept": np.array([d.n_kept for d in diags]),
        "sum_kept": np.array([d.sum_kept for d in diags]),
        "prob": np.array([d.weight / d.sum_kept if d.sum_kept > 0 else np.nan for d in diags]),
    }
