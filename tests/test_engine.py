"""The engine decode-step mirror (lmrs_amd/engine.py): configuration and
strategy mapping on the CPU (generation.rs:71-98, 352-365); the batched
decode step and generation loop on the GPU, against the oracle row by row."""
import numpy as np
import pytest

from lmrs_amd import engine as E
from lmrs_amd import sampling as S


def test_generation_config_validation_and_default():
    c = E.GenerationConfig()
    assert (c.max_tokens, c.temperature, c.top_p, c.top_k) == (128, 1.0, 1.0, None)  # generation.rs:121-130
    assert E.GenerationConfig(32, 0.8, 0.95, 40).max_tokens == 32  # generation.rs:64-67
    for bad in (dict(temperature=0.0), dict(temperature=-1.0), dict(top_p=0.0), dict(top_p=1.5), dict(top_p=-0.1)):
        with pytest.raises(ValueError):
            E.GenerationConfig(**bad)


def test_sampler_for_mapping():
    assert E.sampler_for(E.GenerationConfig(top_k=40, top_p=0.5)) == E.RowParams(40, 1.0, 1.0, True)  # top_k wins
    assert E.sampler_for(E.GenerationConfig(top_p=0.9, temperature=0.7)) == E.RowParams(0, 0.9, 0.7, True)
    assert E.sampler_for(E.GenerationConfig()) == E.RowParams(S.GREEDY, 1.0, 1.0, False)  # Greedy
    assert E.sampler_for(E.GenerationConfig(top_k=1)) == E.RowParams(1, 1.0, 1.0, True)  # TopK(1) draws
    with pytest.raises(S.SamplingError):
        E.sampler_for(E.GenerationConfig(top_k=0))  # TopK::new(0)
    with pytest.raises(S.SamplingError):
        E.sampler_for(E.GenerationConfig(temperature=float("nan")))  # Temperature::new(NaN)


def _decode_vs_oracle(configs, steps=3, V=50000, seed=5):
    """Runs `steps` decode steps of one DecodeBatch over sequences with the
    given GenerationConfigs and compares every step, row by row, with the
    oracle fed the same parameters, histories and uniforms."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helpers import compare, run_oracle
    from lmrs_amd import workloads as W

    S.lib()
    rng = np.random.default_rng(seed)
    seqs = [E.SequenceState(c, seed=11 + i) for i, c in enumerate(configs)]
    batch = E.DecodeBatch(seqs)
    for step in range(steps):
        x = rng.normal(0, 2, (len(seqs), 1, V)).astype(np.float32)
        bits = W.f32_to_bf16_bits(x.reshape(len(seqs), V))
        states = [s.rng for s in seqs]
        # the reference draws one uniform per stochastic row from the Sampler's LCG
        us = []
        for s, st in zip(seqs, states):
            us.append(S.next_unit(st)[0] if s.params.stochastic else 0.0)
        hist = [list(s.generated) for s in seqs]
        logits = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda().reshape(len(seqs), 1, V)
        out = batch.step(logits)
        off = np.concatenate([[0], np.cumsum([len(h) for h in hist])]).astype(np.int64)
        ids = np.concatenate([np.asarray(h, np.uint32) for h in hist] + [np.zeros(0, np.uint32)]).astype(np.uint32)
        B = len(seqs)
        w = W.Workload("engine", bits, np.ones(B, np.float32), np.zeros(B, np.float32), np.zeros(B, np.float32),
                       np.array([s.params.temperature for s in seqs]), np.array([s.params.top_k for s in seqs], np.int32),
                       np.array([s.params.top_p for s in seqs]), np.array(us), off, ids)
        ref = run_oracle(w)
        gpu = {"token_id": np.array([o.token_id for o in out], np.uint32),
               "log_prob": np.array([o.log_prob for o in out], np.float32),
               "logit": np.array([o.logit for o in out], np.float32), "status": np.zeros(B, np.int32)}
        rep = compare(gpu, ref)
        assert rep["token_mismatch"] == 0 and rep["status_mismatch"] == 0 and rep["logit_mismatch"] == 0, rep
        for s, st in zip(seqs, states):  # the RNG advances only for rows that draw
            assert s.rng == (S.next_unit(st)[1] if s.params.stochastic else st)
    return seqs


@pytest.mark.gpu
def test_decode_steps_match_the_oracle_row_by_row():
    _decode_vs_oracle([E.GenerationConfig(8, 1.0, 1.0, None), E.GenerationConfig(8, 0.7, 1.0, 20),
                       E.GenerationConfig(8, 1.3, 0.9, None), E.GenerationConfig(8, 1.0, 0.5, 5),
                       E.GenerationConfig(8, 0.5, 1.0, None)])


@pytest.mark.gpu
def test_wire_params_widened_from_f32_through_decode_steps():
    """Requests carry T and top_p as f32 (openai.rs:160-182); the server widens
    them to f64 (server/engine.rs:115-122), so T = 0.7 samples with
    0.699999988079071 and top_p = 0.9 with 0.8999999761581421.  The decode
    steps must match the oracle fed those widened values."""
    reqs = [{"temperature": 0.7, "top_p": 0.9}, {"temperature": 0.7, "top_k": 40},
            {"temperature": 1.1, "top_p": 0.95}, {"top_p": 0.3}, {"temperature": 0.35},
            {"temperature": 0.7, "top_p": 0.9, "top_k": 1}, {}]
    cfgs = [E.GenerateParams.from_request(r).to_generation_config() for r in reqs]
    assert cfgs[0].temperature == float(np.float32(0.7)) == 0.699999988079071
    assert cfgs[0].top_p == float(np.float32(0.9))
    seqs = _decode_vs_oracle(cfgs, steps=4, V=128256, seed=17)
    assert seqs[0].params.temperature == 0.699999988079071


@pytest.mark.gpu
def test_batched_generate_with_script_models():
    """The ScriptModel of crates/engine/tests/prefill_decode.rs:11-59, three
    sequences at once: one-hot logits at the last position, EOS handling."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    S.lib()
    V = 8
    scripts = [[3, 4, 5], [1, 7, 2], [6, 6, 6, 6]]
    calls = [0, 0, 0]

    def model(step, tokens):
        live = [i for i in range(3) if calls[i] < len(scripts[i]) and not done[i]]
        rows = []
        for i, toks in zip(live, tokens):
            x = torch.zeros(len(toks), V, dtype=torch.bfloat16)
            x[-1, scripts[i][calls[i]]] = 100.0
            calls[i] += 1
            rows.append(x[-1:])
        return torch.stack(rows).cuda()  # [B, 1, V]

    done = [False, False, False]
    cfgs = [E.GenerationConfig(3), E.GenerationConfig(5), E.GenerationConfig(2)]
    seqs = [E.SequenceState(c, eos_token=7) for c in cfgs]
    batch = E.DecodeBatch(seqs)
    step = 0
    while batch.live():
        live = batch.live()
        out = batch.step(model(step, [[0]] * len(live)))
        for i in range(3):
            done[i] = seqs[i].finished
        step += 1
    assert [s.generated for s in seqs] == [[3, 4, 5], [1], [6, 6]]


@pytest.mark.gpu
def test_generate_loop_counts_up():
    """generate() over a batch: a model whose logits favour (last token + 1)
    mod V makes each sequence count up from its prompt's last token; the
    sequence whose count reaches the EOS id stops there."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    S.lib()
    V = 16

    def model(step, tokens):
        x = torch.zeros(len(tokens), 1, V, dtype=torch.bfloat16)
        for j, toks in enumerate(tokens):
            x[j, 0, (toks[-1] + 1) % V] = 50.0
        return x.cuda()

    got = E.generate(model, [[1, 2], [9], [12]], [E.GenerationConfig(4), E.GenerationConfig(3), E.GenerationConfig(6)],
                     eos_token=14)
    assert got == [[3, 4, 5, 6], [10, 11, 12], [13]]


# ---------------------------------------------------------------------------
# the wire format, the sequence state machine and the worker's batch
# ---------------------------------------------------------------------------

def test_generate_params_wire_format():
    # defaults (openai.rs:153-157) and the f32 -> f64 widening of
    # ServerEngine::generate (server/engine.rs:115-122)
    d = E.GenerateParams()
    assert (d.max_tokens, d.temperature, d.top_p, d.top_k, d.stop) == (128, 1.0, 1.0, None, ())
    g = E.GenerateParams(temperature=0.7, top_p=0.9, top_k=40).to_generation_config()
    assert g.temperature == float(np.float32(0.7)) == 0.699999988079071
    assert g.top_p == float(np.float32(0.9)) and g.top_k == 40
    # the widened value is the one the sampler's Temperature holds
    assert E.sampler_for(g).temperature == 0.699999988079071
    r = E.GenerateParams.from_request({"max_tokens": None, "temperature": 0.5, "stop": ["\n"]})
    assert (r.max_tokens, r.temperature, r.top_p, r.top_k, r.stop) == (128, 0.5, 1.0, None, ("\n",))
    # unwrap_or(128) keeps an explicit 0 (openai.rs:160-170)
    assert E.GenerateParams.from_request({"max_tokens": 0}).max_tokens == 0
    with pytest.raises(ValueError):
        E.GenerateParams(temperature=0.0).to_generation_config()


def test_sequence_state_machine():
    O = S.SampleOutput
    # the doctest of sequence.rs:36-47
    seq = E.Sequence(7, [10, 11], 2, 99)
    assert seq.status is E.SequenceStatus.WAITING
    seq.mark_processed(2)
    seq.append_sample(O(12, 0.0, 4.0))
    assert seq.pending_tokens() == [12] and seq.status is E.SequenceStatus.RUNNING
    # EOS is kept and finishes with Eos (sequence.rs:160-172)
    seq.append_sample(O(99, -0.5, 3.0))
    assert seq.generated_token_ids() == [12, 99]
    assert seq.status is E.SequenceStatus.FINISHED and seq.finish_reason is E.FinishReason.EOS
    with pytest.raises(E.SequenceError):
        seq.append_sample(O(1, 0.0, 0.0))
    # Length at max_new_tokens
    s2 = E.Sequence(1, [5], 2)
    s2.append_sample(O(6, 0.0, 0.0))
    s2.append_sample(O(7, 0.0, 0.0))
    assert s2.finish_reason is E.FinishReason.LENGTH and str(s2.finish_reason) == "length"
    with pytest.raises(E.SequenceError):
        E.Sequence(2, [], 4)
    s3 = E.Sequence(3, [1, 2], 4)
    with pytest.raises(E.SequenceError):
        s3.mark_processed(3)
    # status.rs:91-99
    E.validate_transition(E.SequenceStatus.WAITING, E.SequenceStatus.RUNNING)
    with pytest.raises(E.SequenceError):
        E.validate_transition(E.SequenceStatus.FINISHED, E.SequenceStatus.RUNNING)


@pytest.mark.gpu
def test_run_batch_matches_successive_sample_calls():
    """run_batch (one launch) against the reference worker's entry loop: B
    successive Sampler::sample calls on one sampler give the same outputs
    and leave its LCG in the same state, also when an entry fails."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    S.lib()
    rng = np.random.default_rng(5)
    B, V = 12, 4096
    x = torch.from_numpy(rng.normal(0, 2.0, (B, 1, V)).astype(np.float32)).to(torch.bfloat16).cuda()

    def sampler():
        s = S.Sampler(S.SamplerConfig(S.TopK(20)).with_seed(42))
        s.push_processor(S.Temperature(0.8))
        return s

    a, b = sampler(), sampler()
    got = E.run_batch(a, x, list(range(100, 100 + B)))
    want = [b.sample(x[j, -1]) for j in range(B)]
    assert [o.sequence_id for o in got] == list(range(100, 100 + B))
    assert [o.sample for o in got] == want and a.rng == b.rng
    # an entry that fails (a NaN row) stops the batch where the loop stops
    y = x.clone()
    y[5, 0, 7] = float("nan")
    a, b = sampler(), sampler()
    with pytest.raises(S.SamplingError):
        E.run_batch(a, y, list(range(B)))
    with pytest.raises(S.SamplingError):
        for j in range(B):
            b.sample(y[j, -1])
    assert a.rng == b.rng


@pytest.mark.gpu
def test_decode_step_failure_commits_the_other_sequences():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    S.lib()
    V = 4096
    seqs = [E.SequenceState(E.GenerationConfig(8, 1.0, 1.0, 20), seed=7 + i) for i in range(3)]
    batch = E.DecodeBatch(seqs)
    x = torch.randn(3, V).to(torch.bfloat16)
    x[1, 5] = float("nan")  # TopK(20) over a NaN row: invalid distribution (strategies/mod.rs:39-43)
    rngs = [s.rng for s in seqs]
    with pytest.raises(E.BatchSamplingError) as ei:
        batch.step(x.cuda())
    err = ei.value
    assert set(err.errors) == {1} and "invalid probability distribution" in err.errors[1]
    assert seqs[1].rng == rngs[1] and seqs[1].generated == []          # no draw, no token
    for i in (0, 2):                                                  # the others committed
        assert seqs[i].rng == S.next_unit(rngs[i])[1]
        assert len(seqs[i].generated) == 1 and err.outputs[i].token_id == seqs[i].generated[0]
    assert err.outputs[1] is None
