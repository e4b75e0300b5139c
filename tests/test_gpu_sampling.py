"""GPU parity tests: the HIP sampler (through its C-ABI) against the CPU oracle.

Bar: token ids identical except rows where the oracle's uniform lies within
1e-6 of a CDF boundary (or the nucleus cumulative within 1e-6 of top_p, or
exp of a logit at the min-p cut within 1e-12 relative of the threshold),
which are counted; processed logit of the chosen token bit-identical;
post-filter probability exp(log_prob) within 1e-5 relative.
"""
import math

import numpy as np
import pytest

from helpers import assert_parity, compare, run_gpu, run_oracle, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(autouse=True)
def _gpu():
    _require_gpu()
    from lmrs_amd import sampling as S

    S.lib()  # fail loudly if the HIP library is missing


def _wl():
    from lmrs_amd import workloads as W

    return W


def _report(name, rep):
    print(f"[parity] {name}: {rep}", flush=True)


# ---------------------------------------------------------------------------
# the five configurations at their full batch and vocab
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("cfg,rows", [("C1", None), ("C2", None), ("C3", None), ("C4", None), ("C5", None)])
def test_config_parity(cfg, rows):
    W = _wl()
    kw = {"batch": rows} if rows else {}
    if cfg == "C1":
        kw = {"batch": 4}
    w = W.CONFIGS[cfg](**kw)
    print(f"[case] {cfg} B={w.batch} V={w.vocab} {w.dtype}", flush=True)
    rep = compare(run_gpu(w), run_oracle(w))
    _report(cfg, rep)
    assert_parity(rep, cfg)


def test_c1_greedy_check():
    W = _wl()
    w = W.c1(batch=2)
    for k in (-1, 1):  # Greedy, and TopK(1), its softmax_choice twin
        w.top_k[:] = k
        rep = compare(run_gpu(w), run_oracle(w))
        assert_parity(rep, f"C1-greedy k={k}")


def test_c4_contiguous_halves():
    W = _wl()
    w = W.c4(batch=64, layout="halves")
    rep = compare(run_gpu(w), run_oracle(w))
    assert_parity(rep, "C4-halves")


# ---------------------------------------------------------------------------
# processors: exhaustive over all 65536 bf16 patterns
# ---------------------------------------------------------------------------

def test_processors_exhaustive_bf16():
    import oracle as O

    from lmrs_amd import sampling as S

    V = 65536
    allb = np.arange(V, dtype=np.uint32).astype(np.uint16)
    configs = [(1.1, 0.5, 0.3, 0.7), (2.0, 0.0, 0.0, 1.0), (0.7, -1.0, 0.125, 1.5), (1.0, 0.5, 0.25, 1e-3),
               (1.05, 0.0, 0.7, 3.0)]
    # each config runs on 32 rows whose histories (<= 4096 ids each)
    # together mark every pattern once, twice (counts 2) or not at all
    reps = 32
    rows = [(c, o) for c in configs for o in range(reps)]
    B = len(rows)
    x = np.tile(allb, (B, 1))
    hists = [np.concatenate([np.arange(o, V, 2 * reps), np.arange(o, V, 4 * reps), [V + 5]]).astype(np.uint32)
             for _, o in rows]
    off = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    ids = np.concatenate(hists)
    logits = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda()
    out, status = S.process_logits(logits, hist_offsets=torch.from_numpy(off).cuda(),
                                   hist_ids=torch.from_numpy(ids.view(np.int32)).cuda(),
                                   repetition_penalty=[c[0] for c, _ in rows],
                                   presence_penalty=[c[1] for c, _ in rows],
                                   frequency_penalty=[c[2] for c, _ in rows],
                                   temperature=[c[3] for c, _ in rows])
    torch.cuda.synchronize()
    assert np.all(status.cpu().numpy() == 0)
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    for r, ((rep, pres, freq, t), _) in enumerate(rows):
        want = allb.copy()
        want = O.repetition(want, rep, hists[r])[1]
        want = O.presence(want, pres, freq, hists[r])[1]
        want = O.temperature(want, t)[1]
        bad = np.nonzero(got[r] != want)[0]
        assert len(bad) == 0, (rows[r], bad[:8], got[r][bad[:8]], want[bad[:8]])


def test_process_logits_ignores_the_strategy_fields():
    # lmrs_process_logits_fwd is LogitsProcessor::process: an invalid top_p,
    # top_k or min_p in the argument block is neither read nor reported
    import ctypes

    from lmrs_amd import sampling as S

    B, V = 4, 1000
    x = torch.randn(B, V).to(torch.bfloat16).cuda()
    tt = torch.full((B,), 0.7, dtype=torch.float64, device="cuda")
    bad_p = torch.full((B,), 1.5, dtype=torch.float64, device="cuda")
    bad_k = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    status = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    out = torch.empty_like(x)
    args = S.SampleArgs(logits=x.data_ptr(), dtype=S.DTYPE_BF16, batch=B, vocab=V, row_stride=V,
                        temperature=tt.data_ptr(), top_p=bad_p.data_ptr(), top_k=bad_k.data_ptr(),
                        status=status.data_ptr())
    s = torch.cuda.current_stream()
    assert S.lib().lmrs_process_logits_fwd(ctypes.byref(args), ctypes.c_void_p(out.data_ptr()),
                                           ctypes.c_void_p(s.cuda_stream)) == S.LMRS_OK
    torch.cuda.synchronize()
    assert status.cpu().tolist() == [S.ROW_OK] * B
    want, _ = S.process_logits(x, temperature=[0.7] * B)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_sampling_on_a_side_stream_waits_for_its_arguments():
    from lmrs_amd import sampling as S

    W = _wl()
    w = W.c1(batch=4)
    logits = torch.from_numpy(w.logits).cuda()
    side = torch.cuda.Stream()
    ref = run_oracle(w)
    for _ in range(3):  # arguments built on the current stream, launched on the side stream
        res = S.sample_batch(logits, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                             uniforms=w.uniforms, stream=side)
        side.synchronize()
        assert np.array_equal(res["token_ids"].cpu().numpy().view(np.uint32), ref["token_id"])


def test_processors_f32():
    import oracle as O

    from lmrs_amd import sampling as S

    rng = np.random.default_rng(11)
    V = 50000
    x = (rng.standard_normal((3, V)) * 4).astype(np.float32)
    hist = rng.integers(0, V, 700).astype(np.uint32)
    off = np.array([0, 700, 1400, 2100], np.int64)
    ids = np.tile(hist, 3)
    params = [(1.05, 0.0, 0.0, 1.0), (1.3, 0.4, 0.2, 0.8), (0.9, -0.5, 0.1, 2.5)]
    out, _ = S.process_logits(torch.from_numpy(x).cuda(), hist_offsets=torch.from_numpy(off).cuda(),
                              hist_ids=torch.from_numpy(ids.view(np.int32)).cuda(),
                              repetition_penalty=[p[0] for p in params], presence_penalty=[p[1] for p in params],
                              frequency_penalty=[p[2] for p in params], temperature=[p[3] for p in params])
    got = out.cpu().numpy()
    for r, (rep, pres, freq, t) in enumerate(params):
        want = O.temperature(O.presence(O.repetition(x[r], rep, hist)[1], pres, freq, hist)[1], t)[1]
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------------------
# edge cases
# ---------------------------------------------------------------------------

def _mk(logits, **kw):
    """A Workload from explicit rows (numpy float32 or uint16 bf16 bits)."""
    W = _wl()
    B = logits.shape[0]
    f = lambda name, val, dt: np.asarray(kw.get(name, [val] * B), dtype=dt)  # noqa: E731
    hist = kw.get("history")
    off = ids = None
    if hist is not None:
        off = np.concatenate([[0], np.cumsum([len(h) for h in hist])]).astype(np.int64)
        ids = np.concatenate([np.asarray(h, np.uint32) for h in hist]).astype(np.uint32)
    return W.Workload("edge", logits, f("rep", 1.0, np.float32), f("pres", 0.0, np.float32),
                      f("freq", 0.0, np.float32), f("t", 1.0, np.float64), f("k", 0, np.int32),
                      f("p", 1.0, np.float64), f("u", 0.5, np.float64), off, ids,
                      min_p=f("mp", -1.0, np.float64) if "mp" in kw else None)


def test_ties_and_small_rows():
    W = _wl()
    rows = []
    rng = np.random.default_rng(12)
    V = 37
    for _ in range(48):
        rows.append(rng.choice(np.array([0.0, 1.0, 1.0, 2.0, -0.0, 0.5], np.float32), size=V))
    x = np.stack(rows)
    B = len(rows)
    k = rng.choice(np.array([0, 1, 2, 3, 5, 36, 37, 100], np.int32), B)
    p = rng.choice(np.array([1.0, 0.3, 0.5, 0.9, 0.999]), B)
    u = np.concatenate([[0.0, 0.9999999999], rng.random(B - 2)])
    for dt in ("f32", "bf16"):
        xx = x if dt == "f32" else W.f32_to_bf16_bits(x)
        w = _mk(xx, k=k, p=p, u=u)
        rep = compare(run_gpu(w), run_oracle(w))
        _report(f"ties-{dt}", rep)
        assert_parity(rep, dt)


def test_all_equal_row_and_large_tie_groups():
    W = _wl()
    V = 30000
    B = 8
    x = np.zeros((B, V), np.float32)
    x[1::2, ::3] = 1.0  # many tied maxima (10000) on odd rows
    k = np.array([0, 0, 5000, 5000, 12000, 20000, 1, 1], np.int32)
    p = np.array([1.0, 0.5, 1.0, 0.7, 0.95, 0.3, 1.0, 1.0])
    u = np.linspace(0.05, 0.95, B)
    for dt in ("f32", "bf16"):
        xx = x if dt == "f32" else W.f32_to_bf16_bits(x)
        w = _mk(xx, k=k, p=p, u=u)
        rep = compare(run_gpu(w), run_oracle(w))
        _report(f"bigties-{dt}", rep)
        assert_parity(rep, dt)


def test_vocab_sizes_and_unaligned_rows():
    import torch as T

    W = _wl()
    rng = np.random.default_rng(13)
    for V in (1, 2, 3, 7, 8, 9, 1000, 4097, 33333):
        x = (rng.standard_normal((6, V)) * 2).astype(np.float32)
        k = np.array([0, 1, 2, 10, 0, 3], np.int32)
        p = np.array([1.0, 1.0, 0.9, 0.5, 0.8, 1.0])
        for dt in ("f32", "bf16"):
            xx = x if dt == "f32" else W.f32_to_bf16_bits(x)
            w = _mk(xx, k=k, p=p, u=rng.random(6))
            # unaligned rows: a row stride of V + 1 elements, starting one element in
            if xx.dtype == np.uint16:
                big = T.zeros((6, V + 1), dtype=T.int16)
                big[:, 1:] = T.from_numpy(xx.view(np.int16))
                logits = big.view(T.bfloat16).cuda()[:, 1:]
            else:
                big = T.zeros((6, V + 1), dtype=T.float32)
                big[:, 1:] = T.from_numpy(xx)
                logits = big.cuda()[:, 1:]
            ref = run_oracle(w)
            rep = compare(run_gpu(w, logits=logits), ref)
            assert_parity(rep, f"unaligned V={V} {dt}")
            rep = compare(run_gpu(w), ref)
            assert_parity(rep, f"aligned V={V} {dt}")


def test_special_values_and_statuses():
    from lmrs_amd import sampling as S

    V = 16
    x = np.zeros((12, V), np.float32)
    x[0, 3] = np.nan                      # NaN row, sampled -> invalid distribution
    x[1, 3] = np.nan                      # NaN row, Greedy -> the NaN's index
    x[2, 5] = np.inf                      # +inf -> invalid distribution
    x[3, :] = -np.inf                     # all -inf -> invalid distribution
    x[4, :] = -np.inf
    x[4, 7] = 1.0                         # one finite token
    x[5, :] = np.linspace(-3, 3, V)
    x[6, :] = -0.0
    x[6, 2] = 0.0                         # +0 sorts above -0
    x[7, :] = np.linspace(0, 1, V)
    x[8, 5] = np.inf                      # TopK(1) (top_k.rs:39-45) of a +inf maximum: invalid
    x[9, 3] = np.nan                      # TopK(1) of a NaN row: invalid
    x[10, :] = -np.inf                    # TopK(1) of an all -inf row: invalid
    x[11, :] = -np.inf                    # Greedy of an all -inf row: token 0
    k = np.array([0, -1, 0, 0, 0, 0, 1, 0, 1, 1, 1, -1], np.int32)
    p = np.array([1.0, 1.0, 1.0, 1.0, 0.5, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0])
    t = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 0.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0])   # row 5: invalid temperature
    w = _mk(x, k=k, p=p, t=t, u=np.full(12, 0.7))
    g, r = run_gpu(w), run_oracle(w)
    assert list(g["status"] & 0xFF) == list(r["status"]), (g["status"], r["status"])
    assert list(r["status"]) == [2, 0, 2, 2, 0, 3, 0, 0, 2, 2, 2, 0]
    ok = r["status"] == 0
    assert np.array_equal(g["token_id"][ok], r["token_id"][ok])
    # empty vocab
    w0 = _mk(np.zeros((2, 0), np.float32))
    g0 = run_gpu(w0)
    assert list(g0["status"]) == [S.ROW_EMPTY] * 2


def test_history_limits_and_out_of_range_ids():
    """Histories of any length (repetition.rs:88-97 and presence.rs:107-117 have
    no limit): out-of-range ids are ignored; 4096 ids (the fast kernel's
    registers) and 4097 (the generic engine); 20000 ids with about ten
    thousand distinct tokens, and 50000 ids with heavy repeats, through
    the fast kernel's rows (bf16, V % 8 == 0), the generic bf16 engine (odd V)
    and f32 rows; the two table limits report LMRS_ROW_HISTORY."""
    from lmrs_amd import sampling as S

    W = _wl()
    rng = np.random.default_rng(14)
    for V in (128256, 128255):
        # 20000 ids: 9000 distinct tokens once each, then 11000 Zipf(1.1) draws
        zipf = rng.permutation(V)[:9000].tolist() + W._zipf_history(rng, 1, 11000, V)[1].tolist()
        rng.shuffle(zipf)
        assert 9000 < len(set(zipf)) <= S.MAX_HISTORY_DISTINCT
        heavy = list(rng.integers(0, 64, 50000))  # 64 tokens, each ~780 times
        hist = [list(rng.integers(0, V, 100)) + [V, V + 1, 2**32 - 1],   # out-of-range ids ignored
                list(rng.integers(0, V, 4096)),
                list(rng.integers(0, V, 4097)),
                zipf, heavy,
                list(rng.permutation(V)[:S.MAX_HISTORY_DISTINCT + 1]),     # too many distinct tokens
                [7] * (S.MAX_HISTORY_COUNT + 1)]                           # one token too often
        B = len(hist)
        for dt in ("bf16", "f32"):
            x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
            xx = W.f32_to_bf16_bits(x) if dt == "bf16" else x
            w = _mk(xx, history=hist, rep=[1.3] * B, pres=[0.4] * B, freq=[0.2] * B, t=[0.9] * B,
                    k=[0, 40, 0, 0, 50, 40, 40], p=[0.9] * B, u=rng.random(B))
            print(f"[case] histories {dt} V={V} lengths {[len(h) for h in hist]}", flush=True)
            g = run_gpu(w)
            assert list(g["status"][-2:] & 0xFF) == [S.ROW_HISTORY] * 2, g["status"]
            ok = list(range(B - 2))
            r = run_oracle(w.rows(ok))
            sub = {k: v[:B - 2] for k, v in g.items()}
            rep = compare(sub, r)
            _report(f"history-{dt}-{V}", rep)
            assert_parity(rep, f"history-{dt}-{V}")


def test_uniform_extremes():
    W = _wl()
    rng = np.random.default_rng(15)
    V = 2000
    x = W.f32_to_bf16_bits((rng.standard_normal((6, V)) * 2).astype(np.float32))
    u = np.array([0.0, 2.0**-52, 0.5, 1 - 2.0**-52, 1 - 1e-9, 0.25])
    k = np.array([0, 0, 0, 0, 50, 50], np.int32)
    p = np.array([1.0, 0.9, 1.0, 1.0, 0.9, 1.0])
    w = _mk(x, k=k, p=p, u=u)
    rep = compare(run_gpu(w), run_oracle(w))
    assert_parity(rep, "uniforms")


# ---------------------------------------------------------------------------
# the Python mirror of the reference API
# ---------------------------------------------------------------------------

def test_sampler_api_matches_reference_strategies():
    import oracle as O

    from lmrs_amd import sampling as S

    x = torch.tensor([0.0, 10.0, 9.0], dtype=torch.bfloat16).cuda()
    s = S.Sampler(S.SamplerConfig(S.TopK(2)).with_seed(42))
    rng = 42
    for _ in range(6):
        got = s.sample(x, [])
        st, want, rng = O.top_k(np.array([0.0, 10.0, 9.0], np.float32), 2, rng)
        assert got.token_id == want[0]
        assert math.isclose(got.log_prob, want[1], rel_tol=1e-5)
    assert s.rng == rng
    g = S.Sampler()  # default: Greedy, seed 1
    assert g.sample(torch.tensor([0.0, 3.0, 1.0], dtype=torch.bfloat16).cuda()).token_id == 1
    assert g.sample(torch.tensor([1.0, 5.0, 2.0], dtype=torch.bfloat16).cuda()).token_id == 1
    # processors through the mirror
    sp = S.Sampler(S.SamplerConfig(S.TopP(0.9)).with_seed(9))
    sp.push_processor(S.RepetitionPenalty(2.0))
    sp.push_processor(S.Temperature(0.5))
    out = sp.sample(torch.tensor([2.0, -2.0, 1.0, 1.5], dtype=torch.bfloat16).cuda(), [0, 1])
    row = np.array([O.bf16_host(v) for v in [2.0, -2.0, 1.0, 1.5]], np.uint16)
    u, _ = O.next_unit(9)
    st, want, _, _ = O.sample_row(row, [0, 1], O.make_params(repetition_penalty=2.0, temperature=0.5, top_p=0.9), u)
    assert out.token_id == want[0]
    with pytest.raises(S.SamplingError):
        S.Sampler().sample(torch.zeros(0, dtype=torch.bfloat16).cuda())


def test_engine_one_hot_decode_loop():
    from lmrs_amd import sampling as S

    V = 8
    s = S.Sampler()
    got = []
    for tok in (3, 4, 5):  # ScriptModel of crates/engine/tests/prefill_decode.rs:37-84
        row = torch.zeros(1, 1, V, dtype=torch.bfloat16)
        row[0, 0, tok] = 100.0
        got.append(s.sample(row.cuda(), got).token_id)
    assert got == [3, 4, 5]


def test_small_k_bound_and_candidate_paths():
    """Rows that take each branch of the small-k path of the bf16 kernel:
    the coarse second histogram of the thread-value bound (outliers far
    above the rest), the block rank finish (65..512 candidates) and the
    sort finish (more than 512: wide ties at the top), candidate chunks
    beyond a thread's largest one (top values in one thread's slots), and
    argmax chunks holding history tokens."""
    W = _wl()
    rng = np.random.default_rng(77)
    for V in (128256, 32000):
        rows, ks, hists, temps = [], [], [], []
        for case in range(6):
            for _ in range(6):
                x = rng.normal(0.0, 1.0, V).astype(np.float32)
                k, h, t = 50, [], 1.0
                if case == 0:  # outliers: the top kTvBins keys hold fewer than k thread values
                    x[rng.choice(V, 5, replace=False)] = 1000.0
                elif case == 1:  # 100 equal maxima, k = 20: 65..512 candidates
                    x[rng.choice(V, 100, replace=False)] = 20.0
                    k = 20
                elif case == 2:  # 600 equal maxima: more than 512 candidates
                    x[rng.choice(V, 600, replace=False)] = 20.0
                    k = 60
                elif case == 3:  # the top values in one thread's slots (element 8 * (s * 512 + 7) + 3)
                    idx = [8 * (s * 512 + 7) + 3 for s in range(V // 4096)]
                    x[idx] = 8.0 + rng.random(len(idx)).astype(np.float32)
                    k = 10
                elif case == 4:  # history tokens beside the largest values, with temperature
                    top = np.argsort(-x)[:200]
                    h = list((top + rng.integers(-3, 4, 200)).clip(0, V - 1)) + list(rng.integers(0, V, 500))
                    k, t = 40, 0.7
                else:  # Greedy and TopK(1) with a penalised maximum
                    top = int(np.argmax(x))
                    h = [top] * 3 + list(rng.integers(0, V, 100))
                    k = -1 if len(rows) % 2 else 1
                rows.append(x)
                ks.append(k)
                hists.append(h)
                temps.append(t)
        B = len(rows)
        xx = W.f32_to_bf16_bits(np.stack(rows))
        w = _mk(xx, k=np.array(ks, np.int32), t=np.array(temps), rep=[1.3] * B, pres=[0.4] * B, freq=[0.2] * B,
                u=rng.random(B), history=hists)
        print(f"[case] small-k paths V={V} B={B}", flush=True)
        rep = compare(run_gpu(w), run_oracle(w))
        _report(f"small-k-paths-{V}", rep)
        assert_parity(rep, f"small-k-paths-{V}")


def test_min_p_on_every_path():
    """MinP (min_p.rs:39-55) alone and after top-k, before top-p, on every
    selection path: the bf16 kernel's small-k (wave finish), mid-k (sorted
    finish) and full-histogram paths, and the generic engine (bf16 rows of
    odd vocab, f32 rows) with its gathered and weighted paths; plus the
    threshold's overflow, underflow and NaN cases."""
    W = _wl()
    rng = np.random.default_rng(91)
    # (top_k, top_p, min_p): cut combinations
    combos = [(0, 1.0, 0.1), (0, 1.0, 0.01), (0, 1.0, 1e-4), (0, 1.0, 0.0), (0, 1.0, 1.0), (0, 0.9, 0.05),
              (20, 1.0, 0.3), (64, 0.8, 0.02), (50, 1.0, 1e-6), (1000, 1.0, 0.01), (1000, 0.95, 1e-4),
              (5000, 1.0, 0.001), (5000, 1.0, 0.2), (2, 1.0, 0.9), (0, 1.0, -1.0), (1, 1.0, 0.5)]
    for dtype, V in (("bf16", 128256), ("bf16", 32001), ("f32", 32000)):
        rows, ks, ps, mps, hists, temps = [], [], [], [], [], []
        for i, (k, p, mp) in enumerate(combos):
            for j in range(2):
                # normal rows keep thousands of candidates at small min_p, heavy-tailed rows a few
                x = (rng.normal(0.0, 1.0, V) if j == 0 else rng.standard_t(4, V) * 2.0).astype(np.float32)
                h, t = [], 1.0
                if j == 1:  # penalties over a history near the top, with temperature
                    top = np.argsort(-x)[:100]
                    h = list(top[::3]) + list(rng.integers(0, V, 300))
                    t = 0.7
                rows.append(x)
                ks.append(k)
                ps.append(p)
                mps.append(mp)
                hists.append(h)
                temps.append(t)
        # threshold special cases (no history)
        specials = []
        x = rng.normal(0, 1, V).astype(np.float32)
        x[5], x[9] = 800.0, 750.0            # exp overflows: min_p > 0 keeps l >= ~709.8
        specials.append((x, 0, 0.5))
        specials.append((x.copy(), 0, 0.0))  # inf * 0: NaN threshold, empty
        specials.append((x.copy(), 30, 0.5))
        specials.append((x - 2000.0, 0, 0.5))  # exp(max) underflows: everything is kept
        specials.append((x - 2000.0, 40, 0.9))
        y = rng.normal(0, 1, V).astype(np.float32)
        y[77] = np.inf
        specials.append((y, 0, 0.3))          # inf threshold: NaN weights
        specials.append((y.copy(), 0, 0.0))   # NaN threshold
        specials.append((y.copy(), 0, -1.0))  # no min-p: invalid distribution
        specials.append((y.copy(), 5000, -1.0))
        z = rng.normal(0, 1, V).astype(np.float32)
        z[3] = np.nan
        specials.append((z, 0, 0.2))          # NaN maximum: NaN threshold
        for x, k, mp in specials:
            rows.append(x)
            ks.append(k)
            ps.append(1.0)
            mps.append(mp)
            hists.append([])
            temps.append(1.0)
        B = len(rows)
        xx = np.stack(rows)
        if dtype == "bf16":
            xx = W.f32_to_bf16_bits(xx)
        w = _mk(xx, k=np.array(ks, np.int32), p=np.array(ps), mp=np.array(mps), t=np.array(temps),
                rep=[1.2] * B, pres=[0.3] * B, freq=[0.1] * B, u=rng.random(B), history=hists)
        print(f"[case] min-p paths {dtype} V={V} B={B}", flush=True)
        g, r = run_gpu(w), run_oracle(w)
        rep = compare(g, r)
        _report(f"min-p-{dtype}-{V}", rep)
        assert_parity(rep, f"min-p-{dtype}-{V}")
        st = list(r["status"][-len(specials):])
        assert st == [0, 1, 0, 0, 0, 2, 1, 2, 2, 1], st


def test_window_path_cuts_and_fallbacks():
    """The bf16 kernel's top-key window (full distribution and top-k > 64):
    rows it resolves -- top-k and min-p cuts inside it or among the negligible
    elements below it, an isolated maximum, history members inside and below
    it -- and rows it hands to the 65536-bin path: the target, the nucleus
    or the min-p cut below a window whose tail still carries mass."""
    W = _wl()
    rng = np.random.default_rng(123)
    for V in (32000, 128256, 151936):
        rows, ks, ps, mps, ts, us, hists = [], [], [], [], [], [], []

        def add(x, k=0, p=1.0, mp=-1.0, t=1.0, u=None, h=()):
            rows.append(x.astype(np.float32))
            ks.append(k)
            ps.append(p)
            mps.append(mp)
            ts.append(t)
            us.append(rng.random() if u is None else u)
            hists.append(list(h))

        heavy = lambda: rng.standard_t(3, V) * 2.5  # noqa: E731
        normal = lambda s=3.0: rng.normal(0.0, s, V)  # noqa: E731
        add(heavy(), k=1000, t=0.5)                  # k-th token among the negligible elements
        add(heavy(), k=300, p=0.9, t=1.3)            # k-th token inside the window
        add(normal(), k=3000)                        # k-th token inside the window (N(0, 3))
        x = normal(1.0)
        x[rng.integers(V)] = 500.0
        add(x)                                       # an isolated maximum: a one-entry window
        add(normal(), u=0.99995)                     # target below the window: 65536-bin path
        add(normal(1.0), p=0.9999, t=2.0)            # nucleus below the window: 65536-bin path
        add(normal(), mp=1e-9)                       # min-p cut below a window with mass under it
        add(heavy(), mp=1e-30, t=0.5)                # min-p cut among the negligible elements
        add(normal(), p=0.9, mp=0.01, t=0.8)         # min-p and nucleus inside the window
        x = np.full(V, -np.inf)
        x[rng.choice(V, 40, replace=False)] = rng.normal(0, 1, 40)
        add(x, k=200)                                # -inf everywhere but 40 tokens
        top = None
        for t in (1.0, 0.7):                         # members inside and below the window
            x = normal()
            top = np.argsort(-x)[:400]
            add(x, p=0.95, t=t, h=list(top[::2]) + list(rng.integers(0, V, 300)))
        B = len(rows)
        xx = W.f32_to_bf16_bits(np.stack(rows))
        w = _mk(xx, k=np.array(ks, np.int32), p=np.array(ps), mp=np.array(mps), t=np.array(ts), u=np.array(us),
                rep=[1.3] * B, pres=[0.4] * B, freq=[0.2] * B, history=hists)
        print(f"[case] window path V={V} B={B}", flush=True)
        rep = compare(run_gpu(w), run_oracle(w))
        _report(f"window-{V}", rep)
        assert_parity(rep, f"window-{V}")


def test_randomized_rows_every_path():
    """Seeded random rows over the distributions and parameters the paths
    branch on (normal, heavy-tailed, flat, spiked, ties; temperature; top-k
    from 1 to beyond the window; top-p; min-p; histories), against the oracle."""
    W = _wl()
    rng = np.random.default_rng(2024)
    # the last two cases have more rows than the GPU has CUs: rows in rounds
    # (one workgroup per row, and for the widest rows persistent workgroups
    # that take several rows each), NaN rows (the generic engine inside the
    # same workgroup) among them
    for V, B, kinds in ((32000, 160, 6), (128256, 96, 6), (8192, 700, 7), (140000, 320, 7)):
        rows, ks, ps, mps, ts, hists = [], [], [], [], [], []
        for _ in range(B):
            kind = rng.integers(kinds)
            if kind == 0:
                x = rng.normal(0, rng.uniform(0.3, 4.0), V)
            elif kind == 1:
                x = rng.standard_t(rng.uniform(1.5, 5.0), V) * rng.uniform(0.5, 3.0)
            elif kind == 2:
                x = rng.uniform(-1, 1, V) * 0.01          # nearly flat
            elif kind == 3:
                x = rng.normal(0, 1, V)
                x[rng.choice(V, rng.integers(1, 20), replace=False)] += rng.uniform(5, 30)
            elif kind == 4:
                x = rng.integers(-8, 8, V).astype(np.float64) / 2  # wide ties
            elif kind == 5:
                x = rng.gumbel(0, 2.0, V)
            else:
                x = rng.normal(0, 1, V)
                x[rng.integers(V)] = np.nan
            rows.append(x.astype(np.float32))
            ks.append(int(rng.choice([0, 0, -1, 1, 2, 10, 50, 64, 65, 300, 1000, 4096, 5000, V + 3])))
            ps.append(float(rng.choice([1.0, 1.0, rng.uniform(0.05, 1.0), 0.999])))
            mps.append(float(rng.choice([-1.0, -1.0, -1.0, 0.0, rng.uniform(0, 0.5), 10 ** rng.uniform(-12, -1)])))
            ts.append(float(rng.choice([1.0, 1.0, rng.uniform(0.3, 2.5)])))
            hists.append(list(rng.integers(0, V, int(rng.choice([0, 0, 50, 600])))))
        B = len(rows)
        xx = W.f32_to_bf16_bits(np.stack(rows))
        w = _mk(xx, k=np.array(ks, np.int32), p=np.array(ps), mp=np.array(mps), t=np.array(ts),
                rep=rng.uniform(0.8, 1.5, B).astype(np.float32), pres=rng.uniform(-0.5, 1.0, B).astype(np.float32),
                freq=rng.uniform(0, 0.5, B).astype(np.float32), u=rng.random(B), history=hists)
        print(f"[case] randomized V={V} B={B}", flush=True)
        rep = compare(run_gpu(w), run_oracle(w))
        _report(f"randomized-{V}", rep)
        assert_parity(rep, f"randomized-{V}")


def test_randomized_f32_rows_every_path():
    """f32 rows of the two-pass kernel: the distributions its bins and
    sub-buckets branch on (normal, heavy-tailed, flat, spiked, bf16-valued ties,
    masked with -1e9 and -inf, ascending rows whose sample misjudges the
    scale, all equal), with top-k partial bins, min-p partial bins, top-p,
    temperature and histories, against the oracle."""
    W = _wl()
    rng = np.random.default_rng(4242)
    for V, B in ((32000, 128), (256000, 48)):
        rows, ks, ps, mps, ts, hists = [], [], [], [], [], []
        for _ in range(B):
            kind = rng.integers(9)
            if kind == 0:
                x = rng.normal(0, rng.uniform(0.02, 4.0), V)
            elif kind == 1:
                x = rng.standard_t(rng.uniform(1.5, 5.0), V) * rng.uniform(0.5, 3.0)
            elif kind == 2:
                x = rng.uniform(-1, 1, V) * 0.01
            elif kind == 3:
                x = rng.normal(0, 1, V)
                x[rng.choice(V, rng.integers(1, 20), replace=False)] += rng.uniform(5, 30)
            elif kind == 4:
                x = W.bf16_bits_to_f32(W.f32_to_bf16_bits(rng.normal(0, 0.05, V).astype(np.float32)))
            elif kind == 5:
                x = rng.normal(0, 2, V)
                x[rng.random(V) < 0.6] = -1e9
                x[rng.random(V) < 0.1] = -np.inf
            elif kind == 6:
                x = np.sort(rng.normal(0, 2, V))          # the sample sees only the lowest values
            elif kind == 7:
                x = np.full(V, 0.25)
            else:
                x = rng.gumbel(0, 2.0, V)
            rows.append(np.asarray(x, np.float32))
            ks.append(int(rng.choice([0, 0, 0, -1, 1, 2, 10, 50, 1000, 5000, V + 3])))
            ps.append(float(rng.choice([1.0, 0.99, 0.9, rng.uniform(0.05, 1.0), 0.999999])))
            mps.append(float(rng.choice([-1.0, -1.0, -1.0, 0.0, rng.uniform(0, 0.5), 10 ** rng.uniform(-12, -1)])))
            ts.append(float(rng.choice([1.0, 1.0, rng.uniform(0.3, 2.5)])))
            hists.append(list(rng.integers(0, V, int(rng.choice([0, 0, 50, 512])))))
        B = len(rows)
        us = rng.random(B)
        us[:4] = [0.0, 1 - 2.0 ** -52, 0.5, 1e-300]
        w = _mk(np.stack(rows), k=np.array(ks, np.int32), p=np.array(ps), mp=np.array(mps), t=np.array(ts),
                rep=rng.uniform(0.8, 1.5, B).astype(np.float32), pres=rng.uniform(-0.5, 1.0, B).astype(np.float32),
                freq=rng.uniform(0, 0.5, B).astype(np.float32), u=us, history=hists)
        print(f"[case] randomized f32 V={V} B={B}", flush=True)
        rep = compare(run_gpu(w), run_oracle(w))
        _report(f"randomized-f32-{V}", rep)
        assert_parity(rep, f"randomized-f32-{V}")


def test_bf16_special_rows_on_the_window_and_mid_paths():
    """bf16 rows of the fast kernel with +inf, -inf runs, all -inf, and a
    single finite value, under top-k 0, 100, 1000 and 5000 (the window, the
    mid-k and the 65536-bin paths decide them) against the oracle."""
    W = _wl()
    rng = np.random.default_rng(31)
    V = 128256
    rows, ks = [], []
    for k in (0, 100, 1000, 5000):
        x = rng.normal(0, 2, V)
        x[rng.integers(V)] = np.inf                  # invalid distribution
        rows.append(x)
        x = rng.normal(0, 2, V)
        x[rng.choice(V, V // 2, replace=False)] = -np.inf  # half -inf
        rows.append(x)
        rows.append(np.full(V, -np.inf))             # all -inf: invalid distribution
        x = np.full(V, -np.inf)
        x[rng.integers(V)] = 3.0                     # one finite token
        rows.append(x)
        x = np.full(V, 2.0)
        x[rng.choice(V, 7, replace=False)] = 2.5     # seven maxima over a flat row
        rows.append(x)
        ks += [k] * 5
    B = len(rows)
    xx = W.f32_to_bf16_bits(np.stack(rows).astype(np.float32))
    w = _mk(xx, k=np.array(ks, np.int32), p=[0.9 if i % 2 else 1.0 for i in range(B)], u=rng.random(B))
    print(f"[case] bf16 special rows V={V} B={B}", flush=True)
    g, r = run_gpu(w), run_oracle(w)
    rep = compare(g, r)
    _report("bf16-special", rep)
    assert_parity(rep, "bf16-special")
    assert list(r["status"][:5]) == [2, 0, 2, 0, 0], r["status"][:5]
