"""Pins the CPU oracle (oracle/lmrs_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible slip in the restatement (a wrong
shift in the LCG, a reversed tie order, rounding by truncation, a missing
re-rounding step, a cumulative walked from the wrong end, dividing where the
reference multiplies) fails at least one of them:

* the reference's own doctest / test vectors (tests/golden/reference_vectors.json);
* independent arithmetic for the primitives (Python big ints for the LCG,
  torch's bf16 conversion for rounding, float64-exact products for f32 ops);
* brute force on tiny rows (exact inverse CDF at interval midpoints);
* distribution-level checks (chi-square of many draws).
"""
import collections
import json
import math
import os
import struct

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")
VEC = json.load(open(GOLDEN))


def bf(x):
    return np.array([O.bf16_host(v) for v in x], dtype=np.uint16)


def torch_bf16_bits(f32):
    """bf16 bits of float32 values by torch's round-to-nearest-even conversion."""
    t = torch.from_numpy(np.ascontiguousarray(f32, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def f32_of_bf16(b):
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# reference vectors
# ---------------------------------------------------------------------------

def test_reference_greedy_and_beam():
    for v in VEC["greedy"]:
        st, (tok, lp, logit) = O.greedy(v["logits"])
        assert st == O.OK and tok == v["token"] and lp == 0.0 and logit == max(v["logits"])
    for v in VEC["beam"]:
        st, (tok, lp, _) = O.beam(v["logits"], v["width"])
        assert st == O.OK and tok == v["token"] and lp == 0.0
    assert O.beam([1.0, 2.0], 0)[0] == O.ERR_PARAM


def test_reference_stochastic_membership():
    for v in VEC["top_k"]:
        st, (tok, _, _), _ = O.top_k(v["logits"], v["k"], v["rng"])
        assert st == O.OK and tok in v["token_in"]
    for v in VEC["top_p"]:
        st, (tok, _, _), _ = O.top_p(v["logits"], v["p"], v["rng"])
        assert st == O.OK and tok in v["token_in"]
    for v in VEC["min_p"]:
        st, (tok, _, _), _ = O.min_p(v["logits"], v["min_p"], v["rng"])
        assert st == O.OK and tok in v["token_in"]


def test_reference_stochastic_exact_ids():
    # The doctests only assert membership; the exact ids follow from the LCG
    # draw and the two-token distribution [e^0, e^-1] / (1 + e^-1) = [0.731, 0.269].
    p_top = 1.0 / (1.0 + math.exp(-1.0))
    for v, fn in ((VEC["top_k"][0], lambda: O.top_k(v["logits"], v["k"], v["rng"])),
                  (VEC["top_p"][0], lambda: O.top_p(v["logits"], v["p"], v["rng"])),
                  (VEC["min_p"][0], lambda: O.min_p(v["logits"], v["min_p"], v["rng"]))):
        u, _ = O.next_unit(v["rng"])
        st, (tok, lp, _), state = fn()
        want = 1 if u <= p_top else 2
        assert tok == want
        assert math.isclose(lp, math.log(p_top if want == 1 else 1 - p_top), rel_tol=1e-6)
        assert state == O.next_unit(v["rng"])[1]  # exactly one draw consumed


def test_reference_sampler_default_bf16():
    for v in VEC["sampler_default_bf16"]:
        st, (tok, lp, logit), _, _ = O.sample_row(bf(v["logits"]), None, O.make_params(top_k=O.GREEDY), 0.0)
        assert st == O.OK and tok == v["token"] and lp == 0.0


def test_reference_repetition_vector():
    for v in VEC["repetition_penalty"]:
        st, out = O.repetition(bf(v["logits"]), v["penalty"], v["history"])
        vals = f32_of_bf16(out)
        for i, want in v["expect_close"].items():
            assert abs(vals[int(i)] - want) < v["tolerance"]
        # the unchecked middle element: negative logits are multiplied by the penalty
        assert vals[1] == -4.0


def test_reference_presence_vector():
    for v in VEC["frequency_presence_penalty"]:
        st, out = O.presence(bf(v["logits"]), v["presence"], v["frequency"], v["history"])
        vals = f32_of_bf16(out)
        for i, want in v["expect_close"].items():
            assert abs(vals[int(i)] - want) < v["tolerance"]


def test_reference_validation():
    x = bf([1.0, 2.0])
    for v in VEC["validation"]:
        if v["processor"] == "temperature":
            st = O.temperature(x, v["value"])[0]
        elif v["processor"] == "repetition":
            st = O.repetition(x, v["value"], [0])[0]
        else:
            st = O.presence(x, v["value"][0], v["value"][1], [0])[0]
        assert (st == O.OK) == v["ok"], v
    # composed sampler rejects the same values
    assert O.sample_row(x, None, O.make_params(temperature=0.0), 0.5)[0] == O.ERR_PARAM
    assert O.sample_row(x, None, O.make_params(top_p=0.0), 0.5)[0] == O.ERR_PARAM
    assert O.sample_row(x, None, O.make_params(top_p=1.5), 0.5)[0] == O.ERR_PARAM
    assert O.sample_row(x, None, O.make_params(top_k=-2), 0.5)[0] == O.ERR_PARAM
    assert O.top_k([1.0], 0, 1)[0] == O.ERR_PARAM


def test_reference_engine_one_hot_greedy():
    v = VEC["engine_greedy_one_hot"][0]
    got = []
    for t in v["script"]:
        row = np.zeros(v["vocab"], np.float32)
        row[t] = v["hot_value"]
        got.append(O.sample_row(torch_bf16_bits(row), None, O.make_params(top_k=O.GREEDY), 0.0)[1][0])
    assert got == v["tokens"]


def test_empty_rows():
    z = np.zeros(0, np.float32)
    assert O.greedy(z)[0] == O.ERR_EMPTY
    assert O.top_k(z, 3, 1)[0] == O.ERR_EMPTY
    assert O.top_p(z, 0.5, 1)[0] == O.ERR_EMPTY
    assert O.sample_row(z, None, O.make_params(), 0.3)[0] == O.ERR_EMPTY


# ---------------------------------------------------------------------------
# primitives
# ---------------------------------------------------------------------------

def test_next_unit_known_answers():
    # hand recurrence with Python integers: state' = state*A + 1 mod 2^64;
    # (state >> 11) | 0x3FF0... sets the exponent of 1.0, so the mantissa is
    # state bits 11..62 and u = those 52 bits / 2^52 (bit 63 is absorbed)
    A = 6364136223846793005
    for seed in (1, 9, 42, 2**63 + 12345, 2**64 - 1):
        s = seed
        for _ in range(5):
            s_next = (s * A + 1) % 2**64
            want = ((s_next >> 11) & (2**52 - 1)) / 2**52
            u, s = O.next_unit(s)
            assert s == s_next
            assert u == want
            assert 0.0 <= u < 1.0
    # literal values (seed 1): state 6364136223846793006
    assert O.next_unit(1) == (0.6900010319888386, 6364136223846793006)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2**32, size=40000, dtype=np.uint64).astype(np.uint32)
    # add exact ties and values near the overflow threshold
    ties = (rng.integers(0, 2**16, size=20000).astype(np.uint32) << 16) | 0x8000
    edge = np.array([0x7F7F8000, 0x7F7FFFFF, 0xFF7F8000, 0x00008000, 0x00018000, 0x80008000, 0x7F800000], np.uint32)
    u = np.concatenate([u, ties, edge])
    f = u.view(np.float32)
    finite_or_inf = ~np.isnan(f)
    want = torch_bf16_bits(f[finite_or_inf])
    got_h = np.array([O.bf16_host(x) for x in f[finite_or_inf]], np.uint16)
    got_d = np.array([O.bf16_dev(x) for x in f[finite_or_inf]], np.uint16)
    assert np.array_equal(got_h, want)
    assert np.array_equal(got_d, want)
    # ties go to even
    assert O.bf16_dev(struct.unpack("<f", struct.pack("<I", 0x3F808000))[0]) == 0x3F80
    assert O.bf16_dev(struct.unpack("<f", struct.pack("<I", 0x3F818000))[0]) == 0x3F82
    # NaN handling: device canonical, host keeps payload + quiet bit
    nan = struct.unpack("<f", struct.pack("<I", 0xFF812345))[0]
    assert O.bf16_dev(nan) == 0x7FFF
    assert O.bf16_host(nan) == 0xFFC1


def _py_total_key(x):
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    return u ^ 0xFFFFFFFF if u >> 31 else u | 0x80000000


def test_total_cmp_order():
    vals = [-math.inf, -1.0, -0.0, 0.0, 1e-45, 1.0, math.inf]
    for i, a in enumerate(vals):
        for j, b in enumerate(vals):
            assert O.total_cmp(a, b) == (i > j) - (i < j)
    pnan = struct.unpack("<f", struct.pack("<I", 0x7FC00000))[0]
    nnan = struct.unpack("<f", struct.pack("<I", 0xFFC00000))[0]
    assert O.total_cmp(pnan, math.inf) == 1
    assert O.total_cmp(nnan, -math.inf) == -1


def test_sorted_indices_bruteforce():
    rng = np.random.default_rng(1)
    for n in (1, 2, 7, 64, 1000):
        x = rng.choice(np.array([-2.0, -0.0, 0.0, 0.5, 0.5, 3.0, -math.inf], np.float32), size=n)
        got = O.sorted_indices(x)
        want = sorted(range(n), key=lambda i: (-_py_total_key(float(x[i])), i))
        assert list(got) == want


# ---------------------------------------------------------------------------
# strategies and the composed sampler, by brute force
# ---------------------------------------------------------------------------

def _expected_draw(values, order, u):
    """Exact inverse CDF over `order` with weights exp(v - v[order[0]])."""
    m = values[order[0]]
    w = [math.exp(float(np.float32(values[i] - m))) for i in order]
    s = sum(w)
    acc = 0.0
    for i, wi in zip(order, w):
        acc += wi
        if u * s <= acc:
            return i, wi / s
    return order[-1], w[-1] / s


def _midpoints(values, order):
    m = values[order[0]]
    w = np.array([math.exp(float(np.float32(values[i] - m))) for i in order])
    c = np.concatenate([[0.0], np.cumsum(w) / w.sum()])
    return (c[:-1] + c[1:]) / 2


def test_full_draw_bruteforce():
    rng = np.random.default_rng(2)
    for _ in range(60):
        n = int(rng.integers(1, 9))
        x = rng.choice(np.arange(-3, 4, dtype=np.float32) / 2, size=n)  # many ties
        order = sorted(range(n), key=lambda i: (-x[i], i))
        for u in _midpoints(x, order):
            st, (tok, lp, logit), diag, _ = O.sample_row(x, None, O.make_params(), float(u))
            want, prob = _expected_draw(x, order, u)
            assert st == O.OK and tok == want
            assert math.isclose(math.exp(lp), prob, rel_tol=1e-6)
            assert logit == x[want]


def test_top_k_cut_with_ties_bruteforce():
    rng = np.random.default_rng(3)
    for _ in range(60):
        n = int(rng.integers(2, 10))
        k = int(rng.integers(1, n + 2))
        x = rng.choice(np.array([0.0, 1.0, 1.0, 2.0], np.float32), size=n)
        order = sorted(range(n), key=lambda i: (-x[i], i))[: min(k, n)]
        for u in _midpoints(x, order):
            st, (tok, _, _), diag, _ = O.sample_row(x, None, O.make_params(top_k=k), float(u))
            assert tok == _expected_draw(x, order, u)[0]
            assert diag.n_candidates == min(k, n)


def test_top_p_cut_bruteforce():
    rng = np.random.default_rng(4)
    for _ in range(60):
        n = int(rng.integers(2, 9))
        x = rng.normal(size=n).astype(np.float32)
        full = sorted(range(n), key=lambda i: (-x[i], i))
        m = x[full[0]]
        w = np.array([math.exp(float(np.float32(x[i] - m))) for i in full])
        cum = np.cumsum(w) / w.sum()
        j = int(rng.integers(0, n))
        lo = cum[j - 1] if j > 0 else 0.0
        p = float((lo + cum[j]) / 2)  # strictly between cumulative values: cut keeps j+1
        order = full[: j + 1]
        for u in _midpoints(x, order):
            st, (tok, _, _), diag, _ = O.sample_row(x, None, O.make_params(top_p=p), float(u))
            assert st == O.OK and diag.n_kept == j + 1
            assert tok == _expected_draw(x, order, u)[0]


def test_composition_reduces_to_reference_strategies():
    rng = np.random.default_rng(5)
    for trial in range(40):
        n = int(rng.integers(2, 300))
        x = rng.normal(size=n).astype(np.float32) * 3
        seed = int(rng.integers(1, 2**63))
        u, _ = O.next_unit(seed)
        k = int(rng.integers(1, n + 3))
        p = float(rng.uniform(0.05, 1.0))
        _, a, _ = O.top_k(x, k, seed)
        assert O.sample_row(x, None, O.make_params(top_k=k), u)[1] == a
        _, b, _ = O.top_p(x, p, seed)
        assert O.sample_row(x, None, O.make_params(top_p=p), u)[1] == b
        mp = float(rng.choice([0.0, 0.02, 0.3, 1.0, rng.uniform(0.0, 1.0)]))
        st_m, m, _ = O.min_p(x, mp, seed)
        r = O.sample_row(x, None, O.make_params(min_p=mp), u)
        assert r[0] == st_m and r[1] == m
        _, g = O.greedy(x)
        assert O.sample_row(x, None, O.make_params(top_k=O.GREEDY), u)[1] == g
        _, g1, _ = O.top_k(x, 1, seed)
        assert O.sample_row(x, None, O.make_params(top_k=1), u)[1] == g1
        # no filter: full multinomial == TopK(n)
        _, f, _ = O.top_k(x, n, seed)
        assert O.sample_row(x, None, O.make_params(), u)[1] == f


def test_reference_min_p_vector_through_composition():
    # min_p.rs:9-18: MinP(0.1) on [0, 10, 9] with rng 3 picks 1 or 2; the
    # composed sampler with only min-p on is that strategy
    for v in VEC["min_p"]:
        u, _ = O.next_unit(v["rng"])
        st, out, diag, _ = O.sample_row(np.asarray(v["logits"], np.float32), None,
                                        O.make_params(min_p=v["min_p"]), u)
        assert st == O.OK and out[0] in v["token_in"]
        assert out == O.min_p(v["logits"], v["min_p"], v["rng"])[1]
        assert diag.n_kept == 2  # exp(9) >= 0.1 * exp(10) keeps 9; exp(0) does not


def test_min_p_cut_bruteforce():
    # min_p strictly between two consecutive ratios exp(l - max) of distinct
    # values, so the kept set is {l : exp(l - max) >= min_p} whatever exp's
    # last-bit rounding; draws at interval midpoints of the kept prefix
    rng = np.random.default_rng(7)
    for _ in range(80):
        n = int(rng.integers(2, 10))
        x = rng.choice(np.arange(-6, 3, dtype=np.float32) / 2, size=n)
        full = sorted(range(n), key=lambda i: (-x[i], i))
        m = x[full[0]]
        ratios = sorted({math.exp(float(x[i] - m)) for i in range(n)}, reverse=True)
        j = int(rng.integers(0, len(ratios)))
        lo = ratios[j + 1] if j + 1 < len(ratios) else 0.0
        mp = math.sqrt(ratios[j] * lo) if lo > 0 else ratios[j] / 2
        order = [i for i in full if math.exp(float(x[i] - m)) >= ratios[j]]
        for u in _midpoints(x, order):
            st, (tok, lp, _), diag, _ = O.sample_row(x, None, O.make_params(min_p=mp), float(u))
            want, prob = _expected_draw(x, order, u)
            assert st == O.OK and tok == want and diag.n_kept == len(order)
            assert math.isclose(math.exp(lp), prob, rel_tol=1e-6)
        # with a top-k cut first the kept set is the shorter of the two prefixes
        k = int(rng.integers(1, n + 1))
        if k > 1:
            order_k = order[:k]
            for u in _midpoints(x, order_k):
                st, (tok, _, _), diag, _ = O.sample_row(x, None, O.make_params(top_k=k, min_p=mp), float(u))
                assert st == O.OK and tok == _expected_draw(x, order_k, u)[0]


def test_min_p_special_values_and_validation():
    f = lambda *v: np.array(v, np.float32)  # noqa: E731
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    P = O.make_params
    # NaN maximum: NaN threshold keeps nothing (an empty candidate set)
    assert O.sample_row(f(1.0, np.nan, 0.5), None, P(min_p=0.1), 0.3)[0] == O.ERR_EMPTY
    # +inf maximum: inf threshold keeps the overflowing logits, whose weights are NaN
    assert O.sample_row(f(1.0, np.inf, 0.5), None, P(min_p=0.1), 0.3)[0] == O.ERR_DISTRIBUTION
    assert O.sample_row(f(1.0, np.inf, 0.5), None, P(min_p=0.0), 0.3)[0] == O.ERR_EMPTY  # inf * 0
    # exp(800) overflows: min_p 0 gives a NaN threshold, min_p > 0 keeps only l >= ~709.8
    assert O.sample_row(f(800.0, 0.0, 750.0), None, P(min_p=0.0), 0.3)[0] == O.ERR_EMPTY
    st, out, diag, _ = O.sample_row(f(800.0, 0.0, 750.0, 700.0), None, P(min_p=0.5), 0.99)
    assert st == O.OK and diag.n_kept == 2 and out[0] == 0
    # exp(max) underflows to 0: every non-NaN logit is kept
    st, out, diag, _ = O.sample_row(f(-800.0, -801.0), None, P(min_p=0.5), 0.99)
    assert st == O.OK and diag.n_kept == 2 and out[0] == 1
    # a negative NaN sorts last and never passes, so min-p rescues the row
    row = f(1.0, 0.0, 0.5)
    row[1] = neg_nan
    assert O.sample_row(row, None, P(), 0.3)[0] == O.ERR_DISTRIBUTION
    st, out, diag, _ = O.sample_row(row, None, P(min_p=0.0), 0.99)
    assert st == O.OK and diag.n_kept == 2 and out[0] == 2
    # min_p 1 keeps the maximum's ties; min_p 0 keeps -inf (weight 0)
    assert O.sample_row(f(2.0, 2.0, 1.0), None, P(min_p=1.0), 0.3)[1][0] == 0
    assert O.sample_row(f(2.0, 2.0, 1.0), None, P(min_p=1.0), 0.7)[1][0] == 1
    r0 = O.sample_row(f(-np.inf, 1.0, 0.0), None, P(min_p=0.0), 0.9)
    assert r0[2].n_kept == 3 and r0[1] == O.sample_row(f(-np.inf, 1.0, 0.0), None, P(), 0.9)[1]
    assert O.sample_row(f(-np.inf, -np.inf), None, P(min_p=0.5), 0.3)[0] == O.ERR_DISTRIBUTION
    # validation (min_p.rs:27-29); negative is off
    assert O.sample_row(f(1.0, 0.0), None, P(min_p=float("nan")), 0.3)[0] == O.ERR_PARAM
    assert O.sample_row(f(1.0, 0.0), None, P(min_p=1.5), 0.3)[0] == O.ERR_PARAM
    for off in (-0.5, -np.inf):
        assert O.sample_row(f(1.0, 0.0), None, P(min_p=off), 0.6)[1] == O.sample_row(f(1.0, 0.0), None, P(), 0.6)[1]
    # greedy ignores min-p
    assert O.sample_row(f(1.0, np.nan), None, P(top_k=O.GREEDY, min_p=0.5), 0.3)[1][0] == 1


def test_top_k_one_is_greedy_and_k_ge_v_is_full():
    rng = np.random.default_rng(6)
    x = rng.choice(np.array([1.0, 2.0, 2.0, 0.5], np.float32), size=50)
    for u in (0.0, 0.3, 0.999):
        assert O.sample_row(x, None, O.make_params(top_k=1), u)[1][0] == int(np.argmax(x))
        assert O.sample_row(x, None, O.make_params(top_k=O.GREEDY), u)[1][0] == int(np.argmax(x))
        assert O.sample_row(x, None, O.make_params(top_k=50), u)[1] == O.sample_row(x, None, O.make_params(), u)[1]
        assert O.sample_row(x, None, O.make_params(top_k=500), u)[1] == O.sample_row(x, None, O.make_params(), u)[1]


def test_top_p_limits():
    x = np.array([3.0, 1.0, 2.0, 0.0], np.float32)
    for u in (0.0, 0.5, 0.99):
        st, (tok, lp, _), diag, _ = O.sample_row(x, None, O.make_params(top_p=1e-9), u)
        assert tok == 0 and lp == 0.0 and diag.n_kept == 1


def test_chi_square_of_draws():
    x = (np.arange(20, dtype=np.float32) % 7) * 0.4
    params = O.make_params(top_k=12, top_p=0.9)
    counts = collections.Counter()
    probs = {}
    s = 12345
    N = 40000
    for _ in range(N):
        u, s = O.next_unit(s)
        st, (tok, lp, _), _, _ = O.sample_row(x, None, params, u)
        counts[tok] += 1
        probs[tok] = math.exp(lp)
    assert abs(sum(probs.values()) - 1.0) < 1e-5  # post-filter distribution over kept tokens
    chi2 = sum((counts[t] - N * p) ** 2 / (N * p) for t, p in probs.items())
    assert chi2 < 3 * len(probs) + 30


# ---------------------------------------------------------------------------
# processors: exhaustive sweeps over all bf16 inputs
# ---------------------------------------------------------------------------

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _exact_f32_product(a, b):
    """Correctly rounded f32 product of f32 inputs (via the exact f64 product)."""
    return (a.astype(np.float64) * np.float64(b)).astype(np.float32)


@pytest.mark.parametrize("penalty", [1.1, 2.0, 0.7, 1.05, 1e-3, 3.0e38])
def test_repetition_exhaustive(penalty):
    x = ALL_BF16.copy()
    hist = np.arange(0, 65536, 3, dtype=np.uint32)  # every third token penalised
    st, got = O.repetition(x, penalty, list(hist) + [70000, 65536])  # out-of-range ids ignored
    assert st == O.OK
    v = f32_of_bf16(x)
    pf = f32_of_bf16(torch_bf16_bits(np.array([np.float32(1.0) / np.float32(penalty)])))[0]
    nf = f32_of_bf16(torch_bf16_bits(np.array([penalty], np.float32)))[0]
    member = np.zeros(65536, bool)
    member[hist] = True
    fp = np.where(member, pf, np.float32(1.0)).astype(np.float32)
    fn = np.where(member, nf, np.float32(1.0)).astype(np.float32)
    with np.errstate(all="ignore"):
        pos = torch_bf16_bits((v.astype(np.float64) * fp).astype(np.float32))
        neg = torch_bf16_bits((v.astype(np.float64) * fn).astype(np.float32))
    want = np.where(v >= 0, pos, neg)
    nan = np.isnan(v)
    want[nan] = 0x7FFF  # the device conversion's canonical NaN
    assert np.array_equal(got, want)


@pytest.mark.parametrize("presence,frequency", [(0.5, 0.3), (0.5, 0.25), (-1.0, 0.125), (0.0, 0.7)])
def test_presence_exhaustive(presence, frequency):
    rng = np.random.default_rng(7)
    x = ALL_BF16.copy()
    hist = rng.integers(0, 65536, size=5000).astype(np.uint32)
    st, got = O.presence(x, presence, frequency, hist)
    assert st == O.OK
    cnt = collections.Counter(int(t) for t in hist)
    pen = np.zeros(65536, np.float32)
    for t, c in cnt.items():
        pen[t] = np.float32(np.float32(presence) + np.float32(np.float32(frequency) * np.float32(c)))
    penb = f32_of_bf16(torch_bf16_bits(pen))
    v = f32_of_bf16(x)
    with np.errstate(all="ignore"):
        want = torch_bf16_bits((v.astype(np.float64) - penb.astype(np.float64)).astype(np.float32))
    want[np.isnan(v)] = 0x7FFF
    assert np.array_equal(got, want)
    # skip rule: both zero leaves the row bit-identical (NaNs included)
    st, same = O.presence(x, 0.0, 0.0, hist)
    assert np.array_equal(same, x)


@pytest.mark.parametrize("t", [0.7, 0.8, 1.5, 1.0 / 3.0, 1e-30, 1e6])
def test_temperature_exhaustive(t):
    x = ALL_BF16.copy()
    st, got = O.temperature(x, t)
    assert st == O.OK
    s = np.float32(1.0 / t)
    v = f32_of_bf16(x)
    with np.errstate(all="ignore"):
        prod = _exact_f32_product(v, s)  # single rounding, sign of tiny products kept (fma(x, s, 0))
    prod = np.where(prod == 0, np.where(np.signbit(prod) & (v != 0), prod, np.float32(0.0)), prod)
    want = torch_bf16_bits(prod)
    want[np.isnan(v) | np.isnan(prod)] = 0x7FFF
    assert np.array_equal(got, want)
    # T == 1 is skipped: bit-identical
    assert np.array_equal(O.temperature(x, 1.0)[1], x)


def test_f32_processors_have_no_bf16_rounding():
    rng = np.random.default_rng(8)
    x = rng.normal(size=1000).astype(np.float32)
    hist = [1, 1, 5, 7, 7, 7]
    _, r = O.repetition(x, 1.3, hist)
    assert r[1] == (x[1] * np.float32(np.float32(1) / np.float32(1.3)) if x[1] >= 0 else x[1] * np.float32(1.3))
    _, pz = O.presence(x, 0.5, 0.25, hist)
    assert pz[7] == np.float32(x[7] - np.float32(0.5 + 0.25 * 3))
    _, tz = O.temperature(x, 0.7)
    assert np.array_equal(tz, _exact_f32_product(x, np.float32(1 / 0.7)))


def test_processor_order_in_composition():
    # rep then presence then temperature, each rounded: recompute step by step
    x = torch_bf16_bits(np.array([2.5, -1.25, 0.75, 3.0], np.float32))
    hist = [0, 1, 1]
    params = O.make_params(repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.3, temperature=0.7)
    st, _, _, processed = O.sample_row(x, hist, params, 0.5, want_processed=True)
    a = O.repetition(x, 1.3, hist)[1]
    b = O.presence(a, 0.5, 0.3, hist)[1]
    c = O.temperature(b, 0.7)[1]
    assert np.array_equal(processed, f32_of_bf16(c))
    # a different order gives a different row here, so the order is observable
    b2 = O.repetition(O.presence(x, 0.5, 0.3, hist)[1], 1.3, hist)[1]
    assert not np.array_equal(O.temperature(b2, 0.7)[1], c)


def test_invalid_distribution_rows():
    nanrow = np.array([1.0, np.nan, 0.5], np.float32)
    assert O.sample_row(nanrow, None, O.make_params(), 0.3)[0] == O.ERR_DISTRIBUTION
    infrow = np.array([1.0, np.inf, 0.5], np.float32)
    assert O.sample_row(infrow, None, O.make_params(), 0.3)[0] == O.ERR_DISTRIBUTION
    # greedy does not compute weights: the NaN (sorted first) is returned
    assert O.sample_row(nanrow, None, O.make_params(top_k=O.GREEDY), 0.3)[1][0] == 1
    neginf = np.array([-np.inf, -np.inf], np.float32)
    assert O.sample_row(neginf, None, O.make_params(), 0.3)[0] == O.ERR_DISTRIBUTION
    # -inf below the top-k cut does not matter
    mixed = np.array([1.0, -np.inf, 0.0], np.float32)
    assert O.sample_row(mixed, None, O.make_params(), 0.999)[0] == O.OK


def test_top_k_one_is_not_greedy_on_non_finite_rows():
    # TopK(1) draws through softmax_choice (top_k.rs:39-45): a +inf, NaN or
    # all -inf maximum gives the invalid-distribution error and consumes no
    # draw, where Greedy (greedy.rs:22-29) returns the first sorted token
    rows = [np.array([np.inf, 1.0, 0.0], np.float32), np.array([1.0, np.nan, 0.5], np.float32),
            np.array([-np.inf, -np.inf, -np.inf], np.float32), np.array([0.5, np.inf, np.inf], np.float32)]
    for x in rows:
        st_ref, _, state = O.top_k(x, 1, 42)
        assert st_ref == O.ERR_DISTRIBUTION and state == 42  # no draw consumed
        assert O.sample_row(x, None, O.make_params(top_k=1), 0.3)[0] == O.ERR_DISTRIBUTION
        st_g, g = O.greedy(x)
        assert st_g == O.OK
        r = O.sample_row(x, None, O.make_params(top_k=O.GREEDY), 0.3)
        assert r[0] == O.OK and r[1][0] == g[0] and r[1][1] == 0.0
    # finite rows: the same token, log_prob 0 either way
    x = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    a = O.sample_row(x, None, O.make_params(top_k=1), 0.7)
    b = O.sample_row(x, None, O.make_params(top_k=O.GREEDY), 0.7)
    assert a[0] == b[0] == O.OK and a[1] == b[1] and a[1][0] == 1 and a[1][1] == 0.0


# ---------------------------------------------------------------------------
# the LM head's projection (linear_kernel, tensor_ffi.cu:230-258)
# ---------------------------------------------------------------------------

def test_linear_oracle_identity_and_one_hot():
    """With w = I every output is one exact product: y = x.  With one-hot x
    rows, y[r] picks a column of w."""
    import oracle as O
    from lmrs_amd import workloads as W

    rng = np.random.default_rng(3)
    n = 40
    x = W.f32_to_bf16_bits(rng.normal(0, 3, (5, n)).astype(np.float32))
    eye = W.f32_to_bf16_bits(np.eye(n, dtype=np.float32))
    y, _, _ = O.linear_bf16(x, eye)
    assert np.array_equal(y, x)
    w = W.f32_to_bf16_bits(rng.normal(0, 1, (7, n)).astype(np.float32))
    oh = np.zeros((3, n), np.float32)
    oh[0, 4] = oh[1, 0] = oh[2, n - 1] = 1.0
    y2, _, _ = O.linear_bf16(W.f32_to_bf16_bits(oh), w)
    assert np.array_equal(y2, w[:, [4, 0, n - 1]].T)


def test_linear_oracle_sums_in_order():
    """The f32 sum is the sequential one of linear_kernel (acc += x * w over k):
    numpy's float32 accumulate runs the same order; the bf16 output is its
    round to nearest even; sum |x w| against float64."""
    import oracle as O
    from lmrs_amd import workloads as W

    rng = np.random.default_rng(4)
    rows, n_in, n_out = 6, 333, 29
    xb = W.f32_to_bf16_bits(rng.normal(0, 2, (rows, n_in)).astype(np.float32))
    wb = W.f32_to_bf16_bits(rng.normal(0, 0.05, (n_out, n_in)).astype(np.float32))
    y, acc, sa = O.linear_bf16(xb, wb)
    xf, wf = W.bf16_bits_to_f32(xb), W.bf16_bits_to_f32(wb)
    prod = xf[:, None, :] * wf[None, :, :]  # exact in f32 (two 8-bit mantissas)
    seq = np.add.accumulate(prod, axis=2, dtype=np.float32)[:, :, -1]
    assert np.array_equal(acc.view(np.uint32), seq.view(np.uint32))
    assert np.array_equal(y, W.f32_to_bf16_bits(seq))
    assert np.allclose(sa, np.abs(prod.astype(np.float64)).sum(axis=2), rtol=1e-12)
    # a different summation order moves the f32 sum by at most n * 2^-24 * sum |x w|
    alt = prod.astype(np.float64).sum(axis=2)
    assert np.all(np.abs(acc - alt) <= n_in * 2.0 ** -24 * sa)
