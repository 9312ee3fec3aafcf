"""The generation loop (engine.py) on the CPU: the reference's speculative-decoding tests
(Tests/MLXEngineTests/SpeculativeTests.swift) on synthetic logits, prompt-lookup drafts, the CPU
sampler against the oracle's, and InferenceEngine.run over a stand-in model whose next-token logits
are a fixed function of the two tokens its KV "cache" holds before the position (so a wrong prefix
reuse, a skipped or doubled position shows up as different tokens)."""
import numpy as np
import pytest

import engine
import mlxr
import oracle
from engine import CancelToken, GenerationParameters, InferenceEngine, Sampler, XorShift, ngram_propose

GREEDY = GenerationParameters(temperature=0.0, repetition_penalty=1.0)
PLAIN = GenerationParameters(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0)


def onehot(i, V=8):
    return np.array([4.0 if j == i else j * 0.1 for j in range(V)], np.float32)


def verify(rows, draft, params, sampler, stop_after=1 << 30):
    """SpeculativeTests.verify (:10-21)."""
    shaper = Sampler(params, XorShift(1))
    emitted = []

    def emit(t, _ok):
        emitted.append(t)
        return len(emitted) < stop_after
    acc, running = sampler.verify_draft(draft, lambda i: shaper.distribution(np.array(rows[i], np.float32), len(rows[i]), []), emit)
    return emitted, acc, running


def test_greedy_rejects_at_first_mismatch():
    s = Sampler(GREEDY, XorShift(1))
    rows = [onehot(3), onehot(5), onehot(1), onehot(7)]
    assert verify(rows, [3, 5, 2], GREEDY, s) == ([3, 5, 1], 2, True)
    e, acc, _ = verify(rows, [6, 5, 1], GREEDY, s)
    assert e == [3] and acc == 0


def test_greedy_accepts_all_and_adds_bonus():
    s = Sampler(GREEDY, XorShift(1))
    rows = [onehot(3), onehot(5), onehot(1), onehot(7)]
    assert verify(rows, [3, 5, 1], GREEDY, s) == ([3, 5, 1, 7], 3, True)


def test_stops_when_emit_says_so():
    s = Sampler(GREEDY, XorShift(1))
    rows = [onehot(3), onehot(5), onehot(1), onehot(7)]
    e, _, running = verify(rows, [3, 5, 1], GREEDY, s, stop_after=2)
    assert e == [3, 5] and not running


@pytest.mark.parametrize("draft", [0, 2, 5])
def test_sampled_output_follows_target_distribution(draft):
    """SpeculativeTests :63-83 with 40k draws (tolerance 0.012, ~5 sigma at this count)."""
    row = np.array([1.0, 0.2, 2.0, -0.5, 0.7, -np.inf, 1.5, 0.0], np.float32)
    p = np.exp(row - row.max())
    p /= p.sum()
    s = Sampler(PLAIN, XorShift(12345))
    n = 40000
    counts = np.zeros(8)
    for _ in range(n):
        e, acc, _ = verify([row, onehot(0)], [draft], PLAIN, s)
        counts[e[0]] += 1
        if acc == 0:
            assert e[0] != draft
        assert len(e) == (2 if acc == 1 else 1)
    assert counts[5] == 0
    assert np.max(np.abs(counts / n - p)) < 0.012


def test_sampled_second_token_is_conditioned_on_acceptance():
    row0 = np.array([0.5, 1.0, 0.0, -1.0], np.float32)
    row1 = np.array([0.0, -0.5, 1.2, 0.3], np.float32)
    sm = lambda r: np.exp(r - r.max()) / np.exp(r - r.max()).sum()
    s = Sampler(PLAIN, XorShift(777))
    n, first, pair = 40000, 0, np.zeros(4)
    for _ in range(n):
        e, _, _ = verify([row0, row1, row0], [1, 2], PLAIN, s)
        if e[0] != 1:
            continue
        first += 1
        pair[e[1]] += 1
    assert abs(first / n - sm(row0)[1]) < 0.012
    assert np.max(np.abs(pair / first - sm(row1))) < 0.016


def test_xorshift_unit_draw():
    """The unit draw: 24 bits of the low half of next() (Float.random(in: 0..<1)), and the seed-0 rule."""
    a, b = XorShift(0), XorShift(0x9E3779B97F4A7C15)
    for _ in range(5):
        x = a.next()
        assert x == b.next()
    r = XorShift(99)
    s = XorShift(99)
    for _ in range(100):
        u = r.unit()
        assert 0 <= u < 1 and u == np.float32(((s.next() & 0xFFFFFFFF) >> 8) / 16777216.0)


def brute_ngram(history, max_tokens, max_ngram=3, min_ngram=2, window=8192):
    n = len(history)
    for g in range(max_ngram, min_ngram - 1, -1):
        if n <= g:
            continue
        cands = [i for i in range(max(0, n - window), n - g) if history[i:i + g] == history[n - g:]]
        for i in sorted(cands, reverse=True):
            out = history[i + g:min(i + g + max_tokens, n)]
            if out:
                return out
    return []


def test_ngram_propose():
    assert ngram_propose([1, 2, 3, 4, 1, 2, 3], 4) == [4, 1, 2, 3]
    assert ngram_propose([1, 2, 3, 4, 1, 2, 3], 2) == [4, 1]
    assert ngram_propose([5, 6, 7, 9, 6, 7], 3) == [9, 6, 7]      # trigram misses, bigram hits
    assert ngram_propose([1, 2, 3], 4) == []
    assert ngram_propose([1, 2, 1, 2], 0) == []
    assert ngram_propose([7, 7, 7, 7], 2) == [7]                   # latest occurrence first
    rng = np.random.default_rng(4)
    for _ in range(300):
        h = list(rng.integers(0, 4, rng.integers(0, 40)))
        k = int(rng.integers(1, 8))
        assert ngram_propose(h, k) == brute_ngram(h, k), (h, k)
    h = list(rng.integers(0, 3, 200))
    assert ngram_propose(h, 5, search_window=20) == brute_ngram(h, 5, window=20)


@pytest.mark.parametrize("temp,top_k,top_p,min_p,pen", [(0.8, 40, 0.95, 0.0, 1.05), (1.0, 0, 1.0, 0.05, 1.0),
                                                         (0.5, 5, 0.5, 0.0, 1.3), (0.0, 40, 0.95, 0.0, 1.1)])
def test_cpu_sampler_matches_oracle(temp, top_k, top_p, min_p, pen):
    """The engine's CPU sampler against the oracle's restatement of Sampler.distribution."""
    rng = np.random.default_rng(int(temp * 10) + top_k)
    p = GenerationParameters(temperature=temp, top_k=top_k, top_p=top_p, min_p=min_p, repetition_penalty=pen)
    for _ in range(5):
        logits = rng.normal(0, 2, 3000).astype(np.float32)
        recent = rng.integers(0, 3000, 64).astype(np.int32)
        d = Sampler(p, XorShift(1)).distribution(logits.copy(), 3000, list(recent))
        ids, pr = oracle.sample_distribution(logits, recent, temp, top_k, top_p, min_p, pen)
        assert [t for t, _ in d] == list(ids)
        np.testing.assert_allclose([q for _, q in d], pr, rtol=1e-5, atol=1e-7)
    bad = np.full(10, np.nan, np.float32)
    assert Sampler(p, XorShift(1)).distribution(bad, 10, []) is None


# ------------------------------------------------------------------------------ the loop
class FakeModel:
    """Stand-in for mlxr.Transformer: the logits after position p depend on the tokens its cache
    holds at p and p - 1 (written only by the calls that process those positions)."""
    V = 50

    def __init__(self, max_seq=256, chunk=16):
        self.max_seq, self.vocab_size, self.chunk = max_seq, self.V, chunk
        self.cache = np.full(max_seq + 1, -1, np.int64)
        self.sparse = None
        self.prefill_calls = []
        self.rng_seed = None
        self.inflight = []

    def reusable_prefix(self, common, prev):
        return max(0, min(common, self.max_seq))

    def reset_write_tracking(self):
        pass

    def set_sparse(self, s):
        self.sparse = s

    def seed_sampler(self, seed):
        self.rng_seed = seed

    def _row(self, p):
        a, b = int(self.cache[p]), int(self.cache[p - 1]) if p > 0 else 0
        assert a >= 0 and b >= 0, f"position {p} read before it was written"
        r = np.random.default_rng(a * 1000 + b).normal(0, 1, self.V).astype(np.float32)
        r[(a + 1) % self.V] += 3.0   # a strong habit, so sequences repeat and drafts get accepted
        return r

    def _run(self, tokens, offset, is_cancelled):
        for s in range(0, len(tokens), self.chunk):
            if s > 0 and is_cancelled is not None and is_cancelled():
                raise mlxr.EngineError(-7, "cancelled")
            for i, t in enumerate(tokens[s:s + self.chunk]):
                self.cache[offset + s + i] = t

    def forward(self, tokens, offset, all_logits=False, dense=False, is_cancelled=None):
        self._run(list(tokens), offset, is_cancelled)
        if all_logits:
            return np.stack([self._row(offset + i) for i in range(len(tokens))])
        return self._row(offset + len(tokens) - 1)

    def prefill(self, tokens, offset, sample, is_cancelled=None):
        self.prefill_calls.append((offset, len(tokens)))
        self._run(list(tokens), offset, is_cancelled)
        t = int(np.argmax(self._row(offset + len(tokens) - 1)))
        self.cache[offset + len(tokens)] = t
        return t

    def begin_decode_step(self, offset, sample):
        assert len(self.inflight) < 2
        t = int(np.argmax(self._row(offset)))   # the token at `offset` was written by the last step
        self.cache[offset + 1] = t
        st = mlxr.DecodeStep.__new__(mlxr.DecodeStep)
        st.offset = offset
        self.inflight.append((offset, t))
        return st

    def begin_steps(self, tokens, offset, sample):
        assert not self.inflight, "begin_steps needs nothing in flight"
        self._run(list(tokens), offset, None)
        return self.begin_decode_step(offset + len(tokens) - 1, sample)

    def finish(self, step):
        off, t = self.inflight.pop(0)
        assert off == step.offset
        return t


def tokens_of(events):
    return [e[1] for e in events if e[0] == "token"]


def stats_of(events):
    return [e[1] for e in events if e[0] == "finished"][0]


def test_engine_gpu_sampled_and_speculative_agree():
    prompt = list(np.random.default_rng(1).integers(0, 50, 40))
    a = InferenceEngine(FakeModel()).generate(prompt, GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=60))
    eng = InferenceEngine(FakeModel())
    b = eng.generate(prompt, GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=60, speculative=True))
    assert tokens_of(a) == tokens_of(b) and len(tokens_of(a)) == 60
    sa, sb = stats_of(a), stats_of(b)
    assert sa.stop_reason == sb.stop_reason == "length" and sa.generated_tokens == 60
    assert sb.draft_tokens and sb.accepted_draft_tokens > 10
    assert a[0][0] == "promptProcessed" and a[0][1].prompt_tokens == 40


def test_engine_prefix_reuse_and_stop():
    m = FakeModel()
    eng = InferenceEngine(m)
    prompt = list(np.random.default_rng(2).integers(0, 50, 30))
    first = tokens_of(eng.generate(prompt, GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=10)))
    follow = prompt + first + [7, 8, 9]
    ev = eng.generate(follow, GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=10))
    st = stats_of(ev)
    assert st.cached_prompt_tokens >= 30 and m.prefill_calls[-1][0] == st.cached_prompt_tokens
    fresh = InferenceEngine(FakeModel()).generate(follow, GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=10))
    assert tokens_of(ev) == tokens_of(fresh) and stats_of(fresh).cached_prompt_tokens == 0
    # a stop id ends the reply without being emitted
    stop = tokens_of(fresh)[3]
    eng2 = InferenceEngine(FakeModel(), stop_ids=[stop])
    ev2 = eng2.generate(follow, GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=10))
    assert tokens_of(ev2) == tokens_of(fresh)[:tokens_of(fresh).index(stop)] and stats_of(ev2).stop_reason == "stop"


def test_engine_context_and_cancel():
    m = FakeModel(max_seq=48)
    ev = InferenceEngine(m).generate(list(range(40)), GenerationParameters(temperature=0, repetition_penalty=1, max_tokens=100))
    assert stats_of(ev).stop_reason == "length" and len(tokens_of(ev)) == 8   # max_new = max_seq - prompt
    # cancelled between prefill chunks: no token, reason "cancelled"
    tok = CancelToken()
    calls = []
    m2 = FakeModel()
    orig = m2._run

    def run(tokens, offset, is_cancelled):
        calls.append(1)
        tok.cancel()
        return orig(tokens, offset, is_cancelled)
    m2._run = run
    ev = InferenceEngine(m2).generate(list(range(40)), GenerationParameters(temperature=0, max_tokens=5), tok)
    assert tokens_of(ev) == [] and stats_of(ev).stop_reason == "cancelled"
    # cancelled mid-stream: stops promptly
    tok = CancelToken()
    seen = []

    def emit(e):
        seen.append(e)
        if e[0] == "token" and len(tokens_of(seen)) == 5:
            tok.cancel()
    InferenceEngine(FakeModel()).run(list(range(10)), GenerationParameters(temperature=0, max_tokens=200), tok, emit)
    assert stats_of(seen).stop_reason == "cancelled" and len(tokens_of(seen)) < 8


def test_engine_sampled_is_seeded():
    p = GenerationParameters(temperature=0.9, top_k=20, seed=5, speculative=True)
    a = tokens_of(InferenceEngine(FakeModel()).generate(list(range(12)), dataclasses_replace(p, max_tokens=30)))
    b = tokens_of(InferenceEngine(FakeModel()).generate(list(range(12)), dataclasses_replace(p, max_tokens=30)))
    assert a == b and len(a) == 30


def dataclasses_replace(p, **kw):
    import dataclasses
    return dataclasses.replace(p, **kw)
