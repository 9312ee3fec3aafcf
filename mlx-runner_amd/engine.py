"""The generation loop above the C ABI: `InferenceEngine.run` (Engine.swift:549-813) on token ids.

What it keeps from the reference, on the same `Transformer` calls (mlxr.py over include/mlxr.h):
- prefix reuse with the previous request (Engine.swift:558-564): the common prefix of the cached
  and the new token ids, clamped by `reusable_prefix`; only the rest is prefilled;
- cancellation through a `CancelToken`, polled between prefill chunks (the C ABI's
  `mlxr_cancel_fn`) and before every emitted token;
- plain decoding with the token selected on the GPU, each step committed before the previous one
  is read back (Engine.swift:719-746);
- CPU sampling when decoding speculatively: prompt-lookup drafts (`ngram_propose`,
  Engine.swift:214-235) and drafts from an optional draft model (Engine.swift:619-669), verified in
  one batched pass of up to 8 tokens (`Transformer.forward(all_logits=True)`) with exact
  acceptance (`Sampler.verify_draft`, Engine.swift:180-211);
- `GenerationStats` (Engine.swift:18-40) and the stop reasons "stop", "length", "context",
  "cancelled".

Events go to `emit` as ("promptProcessed", stats), ("token", id) and ("finished", stats): token ids
stand where the reference emits detokenised text (the tokenizer is not part of this library).
"""
from __future__ import annotations

import dataclasses
import threading
import time
from typing import Callable, List, Optional, Sequence, Tuple

import numpy as np

import mlxr

MAX_VERIFY_TOKENS = 8   # Transformer.maxVerifyTokens: rows of one batched verify pass

Dist = List[Tuple[int, float]]


@dataclasses.dataclass
class GenerationParameters(mlxr.SamplingParameters):
    """SamplingParameters (Engine.swift:3-16): the sampler's fields plus the request's."""
    max_tokens: int = 4096
    seed: Optional[int] = None
    speculative: Optional[bool] = None


@dataclasses.dataclass
class GenerationStats:
    """GenerationStats (Engine.swift:18-40)."""
    prompt_tokens: int = 0
    cached_prompt_tokens: int = 0
    generated_tokens: int = 0
    time_to_first_token: float = 0.0
    prompt_tokens_per_second: float = 0.0
    tokens_per_second: float = 0.0
    stop_reason: str = ""
    draft_tokens: Optional[int] = None
    accepted_draft_tokens: Optional[int] = None
    model_draft_tokens: Optional[int] = None
    accepted_model_draft_tokens: Optional[int] = None
    draft_cycles: Optional[int] = None
    draft_seconds: Optional[float] = None
    verify_seconds: Optional[float] = None


class CancelToken:
    """A request's cancel flag (set from any thread)."""

    def __init__(self):
        self._ev = threading.Event()

    def cancel(self):
        self._ev.set()

    @property
    def is_cancelled(self) -> bool:
        return self._ev.is_set()


class XorShift:
    """Engine.swift:95-102: xorshift64, seed 0 replaced by 0x9E3779B97F4A7C15."""
    M = (1 << 64) - 1

    def __init__(self, seed: int):
        self.state = (seed & self.M) or 0x9E3779B97F4A7C15

    def next(self) -> int:
        s = self.state
        s ^= (s << 13) & self.M
        s ^= s >> 7
        s ^= (s << 17) & self.M
        self.state = s
        return s

    def unit(self) -> np.float32:
        """Float.random(in: 0..<1, using:) as Swift's standard library computes it: 24 random bits
        from next(upperBound: 1 << 24) (Lemire's multiply on the low 32 bits of next(), which for a
        power-of-two bound is those bits >> 8, never rejected), times 2^-24."""
        return np.float32(((self.next() & 0xFFFFFFFF) >> 8) * (2.0 ** -24))


class Sampler:
    """Sampler (Engine.swift:105-211): the CPU twin of the GPU token selection, used when decoding
    speculatively. Float32 arithmetic in the reference's order (sequential sums)."""

    def __init__(self, params: mlxr.SamplingParameters, rng: XorShift):
        self.params = params
        self.rng = rng

    def distribution(self, logits: np.ndarray, count: int, recent: Sequence[int]) -> Optional[Dist]:
        """Engine.swift:112-164. `logits` is modified in place (the repetition penalty), as there."""
        p = self.params
        row = logits[:count]
        if p.repetition_penalty != 1 and len(recent):
            pen = np.float32(p.repetition_penalty)
            for t in set(int(t) for t in recent):
                if 0 <= t < count:
                    row[t] = row[t] / pen if row[t] > 0 else row[t] * pen
        if p.temperature <= 0.001:
            # strict > from index 0: the lowest index among equal maxima; NaN never wins
            finite_or_inf = np.where(np.isnan(row), -np.inf, row)
            best = int(np.argmax(finite_or_inf))
            v = finite_or_inf[best]
            if v == -np.inf:
                best = 0
            return [(best, 1.0)] if np.isfinite(v) else None
        k = min(p.top_k, count) if p.top_k > 0 else min(512, count)
        # the k largest by value, descending; among equal values the lower index first (the
        # reference's insertion keeps arrival order for ties)
        order = np.argsort(-row.astype(np.float64), kind="stable")[:k]
        vals = row[order]
        max_v = vals[0]
        if not np.isfinite(max_v):
            return None
        inv_t = np.float32(1.0) / np.float32(p.temperature)
        probs = np.exp((vals - max_v) * inv_t).astype(np.float32)
        total = np.cumsum(probs, dtype=np.float32)[-1]
        cut = len(probs)
        if p.min_p > 0:
            below = np.nonzero(probs < np.float32(p.min_p) * probs[0])[0]
            if below.size:
                cut = int(below[0])
        if p.top_p < 1:
            acc = np.cumsum(probs[:cut] / total, dtype=np.float32)
            hit = np.nonzero(acc >= np.float32(p.top_p))[0]
            if hit.size:
                cut = int(hit[0]) + 1
        cut = max(1, cut)
        total = np.cumsum(probs[:cut], dtype=np.float32)[-1]
        return [(int(order[i]), float(probs[i] / total)) for i in range(cut)]

    def draw(self, dist: Dist) -> int:
        """Engine.swift:166-173."""
        r = self.rng.unit()
        for tid, pr in dist:
            r = np.float32(r - np.float32(pr))
            if r <= 0:
                return tid
        return dist[-1][0]

    def verify(self, dist: Dist, draft: int) -> Tuple[bool, int]:
        """Exact acceptance of a deterministic draft (Engine.swift:178-187): accept with p(draft),
        otherwise draw from p with the draft removed."""
        pd = next((pr for tid, pr in dist if tid == draft), 0.0)
        if pd >= 1 or (pd > 0 and self.rng.unit() < np.float32(pd)):
            return True, draft
        rest = [(tid, pr) for tid, pr in dist if tid != draft]
        total = np.float32(0)
        for _, pr in rest:
            total = np.float32(total + np.float32(pr))
        if not total > 0:
            return True, draft
        return False, self.draw([(tid, float(np.float32(pr) / total)) for tid, pr in rest])

    def verify_draft(self, draft: Sequence[int], dist: Callable[[int], Dist],
                     emit: Callable[[int, bool], bool]) -> Tuple[int, bool]:
        """Engine.swift:195-211: drafts in order; the first rejection emits its correction; all
        accepted adds the last row's bonus token. Returns (accepted drafts, still running)."""
        accepted = 0
        for i, d in enumerate(draft):
            ok, t = self.verify(dist(i), d)
            if ok:
                accepted += 1
            if not emit(t, ok):
                return accepted, False
            if not ok:
                return accepted, True
        return accepted, emit(self.draw(dist(len(draft))), False)


def ngram_propose(history: Sequence[int], max_tokens: int, max_ngram: int = 3, min_ngram: int = 2,
                  search_window: int = 8192) -> List[int]:
    """Prompt-lookup drafts (NGramDraft.propose, Engine.swift:214-235): the tokens that followed the
    latest earlier occurrence of the history's last g tokens (g from max_ngram down to min_ngram)."""
    if max_tokens <= 0:
        return []
    n = len(history)
    lo = max(0, n - search_window)
    h = list(history)
    for g in range(max_ngram, min_ngram - 1, -1):
        if n <= g:
            continue
        tail = n - g
        pat = h[tail:]
        for i in range(tail - 1, lo - 1, -1):
            if h[i:i + g] == pat:
                start = i + g
                end = min(start + max_tokens, n)
                if end > start:
                    return h[start:end]
    return []


class InferenceEngine:
    """A loaded model (and an optional draft model of the same vocabulary) with the prompt cache of
    the previous request."""

    def __init__(self, model: mlxr.Transformer, stop_ids: Sequence[int] = (), draft_model: Optional[mlxr.Transformer] = None):
        self.model = model
        self.stop_ids = set(int(t) for t in stop_ids)
        self.draft_model = draft_model
        self.cached_tokens: List[int] = []
        self.draft_cached: List[int] = []

    def generate(self, tokens: Sequence[int], parameters: GenerationParameters, token: Optional[CancelToken] = None):
        """The events of one request as a list (run() with a collecting emit)."""
        events = []
        self.run(tokens, parameters, token or CancelToken(), events.append)
        return events

    def run(self, tokens: Sequence[int], parameters: GenerationParameters, token: CancelToken, emit: Callable) -> None:
        model = self.model
        tokens = [int(t) for t in tokens]
        stats = GenerationStats(prompt_tokens=len(tokens))
        if not tokens:
            raise mlxr.EngineError(-2, "Empty prompt")
        if len(tokens) >= model.max_seq:
            raise mlxr.EngineError(-5, "The context window is full.")

        # reuse the KV cache for the prefix shared with the previous request (Engine.swift:558-564)
        common = 0
        limit = min(len(self.cached_tokens), len(tokens) - 1)
        while common < limit and self.cached_tokens[common] == tokens[common]:
            common += 1
        common = model.reusable_prefix(common, len(self.cached_tokens))
        if common == 0:
            model.reset_write_tracking()
        stats.cached_prompt_tokens = common

        vocab = model.vocab_size
        seed = parameters.seed if parameters.seed is not None else int.from_bytes(np.random.bytes(8), "little") or 1
        draft_model = self.draft_model if parameters.speculative is not False else None
        prompt_lookup = bool(parameters.speculative) or draft_model is not None
        speculative = prompt_lookup or draft_model is not None
        gpu_sampling = not speculative
        model_sparse = model.sparse
        if speculative:   # verification passes are dense, and so is every step of the request
            model.set_sparse(None)
        try:
            self._run(tokens, parameters, token, emit, stats, common, vocab, seed, draft_model, prompt_lookup,
                      speculative, gpu_sampling)
        finally:
            if speculative and model_sparse is not None:
                model.set_sparse(model_sparse)

    def _run(self, tokens, parameters, token, emit, stats, common, vocab, seed, draft_model, prompt_lookup,
             speculative, gpu_sampling):
        model = self.model
        count = vocab
        self.cached_tokens = tokens[:common]
        draft_ok = draft_model is not None
        if draft_model is not None:
            dc = 0
            dl = min(len(self.draft_cached), len(tokens) - 1)
            while dc < dl and self.draft_cached[dc] == tokens[dc]:
                dc += 1
            dc = draft_model.reusable_prefix(dc, len(self.draft_cached))
            if dc == 0:
                draft_model.reset_write_tracking()
            self.draft_cached = tokens[:dc]

        t0 = time.perf_counter()
        logits = None
        first_token = None
        cancelled = lambda: token.is_cancelled
        try:
            prompt = tokens[common:]
            if gpu_sampling:
                model.seed_sampler(seed)
                first_token = model.prefill(prompt, common, parameters, is_cancelled=cancelled)
            else:
                logits = model.forward(prompt, common, dense=True, is_cancelled=cancelled)
        except mlxr.EngineError as e:
            if e.case != "cancelled":
                raise
            stats.stop_reason = "cancelled"
            emit(("finished", stats))
            return
        history = list(tokens)
        self.cached_tokens = list(tokens)
        t_prompt = time.perf_counter() - t0
        stats.time_to_first_token = t_prompt
        stats.prompt_tokens_per_second = (len(tokens) - common) / max(t_prompt, 1e-6)
        emit(("promptProcessed", dataclasses.replace(stats)))

        sampler = Sampler(parameters, XorShift(seed))
        shaper = Sampler(parameters, XorShift(seed))   # builds distributions only (no draws)
        t_gen = time.perf_counter()
        stats.stop_reason = "length"
        max_new = min(parameters.max_tokens, model.max_seq - len(tokens))
        drafted = accepted_drafts = 0
        draft_len = 4
        greedy_draft = dataclasses.replace(parameters, temperature=0.0)
        draft_checked = len(self.draft_cached)
        model_draft_len = 4
        model_drafted = model_accepted = model_cycles = 0
        draft_time = verify_time = 0.0

        def accept(t: int) -> bool:
            if t in self.stop_ids:
                stats.stop_reason = "stop"
                return False
            stats.generated_tokens += 1
            emit(("token", t))
            history.append(t)
            if stats.generated_tokens >= max_new:
                stats.stop_reason = "length"
                return False
            if len(history) >= model.max_seq:
                stats.stop_reason = "context"
                return False
            return True

        def dist(row: np.ndarray) -> Dist:
            d = shaper.distribution(row, count, history[-parameters.repetition_window:] if parameters.repetition_window > 0 else [])
            if d is None:
                raise mlxr.EngineError(-8, "non-finite logits")
            return d

        def propose_from_model(k: int) -> List[int]:
            """Engine.swift:619-669: up to k greedy tokens of the draft model after the pending one."""
            nonlocal draft_checked, draft_ok, draft_time
            d = draft_model
            if d is None or not draft_ok:
                return []
            P = len(history) - 1
            keep = min(draft_checked, len(self.draft_cached))
            lim = min(len(self.draft_cached), P)
            while keep < lim and self.draft_cached[keep] == history[keep]:
                keep += 1
            del self.draft_cached[keep:]
            k = min(k, d.max_seq - 1 - P)
            if k <= 0:
                return []
            start = time.perf_counter()
            try:
                catch_up = history[keep:]
                out: List[int] = []
                if len(catch_up) > 16:   # after long prompt-lookup runs only
                    out.append(d.prefill(catch_up, keep, greedy_draft))
                    inflight = d.begin_decode_step(P + 1, greedy_draft) if k > 1 else None
                else:
                    inflight = d.begin_steps(catch_up, keep, greedy_draft)
                self.draft_cached = list(history)
                draft_checked = P + 1
                # the next step is queued before the current one is read back (two in flight)
                while inflight is not None:
                    cur, inflight = inflight, None
                    if cur.offset + 1 < P + k:
                        try:
                            inflight = d.begin_decode_step(cur.offset + 1, greedy_draft)
                        except mlxr.EngineError:
                            _try_finish(d, cur)
                            raise
                    try:
                        out.append(d.finish(cur))
                    except mlxr.EngineError:
                        if inflight is not None:
                            _try_finish(d, inflight)
                        raise
                self.draft_cached += out[:-1]   # the last draft was never processed
                draft_time += time.perf_counter() - start
                return out
            except mlxr.EngineError:
                self.draft_cached = history[:keep]
                draft_checked = keep
                draft_ok = False
                return []

        running = max_new > 0 and not token.is_cancelled
        if first_token is not None:
            # GPU sampling: the step of the newest token is committed before the previous one is read
            if running:
                running = accept(first_token)
            cached_count = len(tokens)
            inflight = model.begin_decode_step(len(history) - 1, parameters) if running else None
            while inflight is not None:
                cur, inflight = inflight, None
                nxt = cur.offset + 1
                if not token.is_cancelled and stats.generated_tokens + 1 < max_new and nxt + 1 < model.max_seq:
                    try:
                        inflight = model.begin_decode_step(nxt, parameters)
                    except mlxr.EngineError:
                        _try_finish(model, cur)
                        raise
                try:
                    t = model.finish(cur)
                except mlxr.EngineError:
                    if inflight is not None:
                        _try_finish(model, inflight)
                    raise
                cached_count = cur.offset + 1
                if token.is_cancelled:
                    stats.stop_reason = "cancelled"
                    break
                if not accept(t):
                    break
            if inflight is not None and _try_finish(model, inflight):
                cached_count = inflight.offset + 1
            self.cached_tokens = history[:min(len(history), cached_count)]
            running = False

        # CPU sampling (speculative decoding): history[-1] is pending (not in the KV cache yet)
        if running and logits is not None:
            running = accept(sampler.draw(dist(logits)))
        while running:
            if token.is_cancelled:
                stats.stop_reason = "cancelled"
                break
            pending = history[-1]
            room = min(max_new - stats.generated_tokens, model.max_seq - len(history)) - 1
            cap = min(room, MAX_VERIFY_TOKENS - 1) if speculative else 0
            draft = ngram_propose(history, min(draft_len, cap)) if prompt_lookup else []
            from_model = not draft and cap > 0 and draft_ok
            if from_model:
                draft = propose_from_model(min(model_draft_len, cap))
            if not draft:
                row = model.forward([pending], len(history) - 1)
                self.cached_tokens = list(history)
                running = accept(sampler.draw(dist(row)))
                continue
            t_verify = time.perf_counter()
            rows = model.forward([pending] + draft, len(history) - 1, all_logits=True)
            self.cached_tokens = list(history)
            drafted += len(draft)

            def emit_tok(t, ok):
                r = accept(t)
                if ok and r:
                    self.cached_tokens = list(history)
                return r
            acc, running = sampler.verify_draft(draft, lambda i: dist(rows[i]), emit_tok)
            accepted_drafts += acc
            if from_model:
                verify_time += time.perf_counter() - t_verify
                model_cycles += 1
                model_drafted += len(draft)
                model_accepted += acc
                model_draft_len = (min(model_draft_len + 1, MAX_VERIFY_TOKENS - 1) if acc == len(draft)
                                   else max(1, model_draft_len - 1) if acc == 0 else model_draft_len)
            else:
                draft_len = min(draft_len + 1, MAX_VERIFY_TOKENS - 1) if acc == len(draft) else max(1, acc)

        dt = time.perf_counter() - t_gen
        stats.tokens_per_second = stats.generated_tokens / max(dt, 1e-6)
        if drafted > 0:
            stats.draft_tokens, stats.accepted_draft_tokens = drafted, accepted_drafts
        if draft_model is not None:
            stats.model_draft_tokens, stats.accepted_model_draft_tokens = model_drafted, model_accepted
        if model_cycles > 0:
            stats.draft_cycles, stats.draft_seconds, stats.verify_seconds = model_cycles, draft_time, verify_time
        emit(("finished", stats))


def _try_finish(model, step) -> bool:
    try:
        model.finish(step)
        return True
    except mlxr.EngineError:
        return False
