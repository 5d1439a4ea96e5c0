"""Greedy generation with n-gram speculative decoding (rich_triplet_amd.generate):
the drafter against the reference's own test, the greedy pick, the loop's
bookkeeping on a toy context and on the oracle model, and on the GPU the
speculative run (batched verify, rejected drafts overwritten in the cache)
against the plain one."""
from __future__ import annotations

import copy

import numpy as np
import pytest

from test_gpu_decode import tiny
from test_oracle import make_model


def test_ngram_draft_engine_reference_case(rt):
    """transformer4.rs:3456-3489 (test_ngram_draft_engine), step by step."""
    ng = rt.NgramDraftEngine(4, 4)
    assert ng.draft() == []
    for t in [10, 20, 30, 40, 10, 20, 30, 40, 50, 60]:
        ng.record(t)
    assert ng.draft() == []
    ng.record(10)
    assert ng.draft() == []
    ng.record(20)
    assert ng.draft() == [30, 40, 10, 20]


def test_ngram_draft_engine_rules(rt):
    ng = rt.NgramDraftEngine(4, 3)
    ng.record_many([1, 2, 3, 9, 1, 2, 3, 7, 5, 1, 2, 3])
    # the longest suffix first: [2, 3] would match earlier, but [1, 2, 3] at 0 wins
    assert ng.draft() == [9, 1, 2]
    # max_draft caps the continuation; the history end caps it too
    ng = rt.NgramDraftEngine(2, 8)
    ng.record_many([4, 5, 6, 4, 5])
    assert ng.draft() == [6, 4, 5]
    # max_draft 0: every match has an empty continuation
    ng = rt.NgramDraftEngine(4, 0)
    ng.record_many([4, 5, 4, 5])
    assert ng.draft() == []
    # one token of history drafts nothing
    ng = rt.NgramDraftEngine(4, 4)
    ng.record(3)
    assert ng.draft() == []


def test_greedy_token_picks_last_of_equal_maxima(rt):
    assert rt.greedy_token(np.array([0.5, 2.0, 1.0], np.float32)) == 1
    assert rt.greedy_token(np.array([3.0, 1.0, 3.0, 2.0], np.float32)) == 2
    # probabilities that round to the same f32 tie as well (exp(-2^-30) == 1)
    assert rt.greedy_token(np.array([1.0, 1.0 - 2.0 ** -30, 0.0], np.float32)) == 1


class ToyCtx:
    """A deterministic toy model with a KV cache: the next token is a fixed
    function of the cached tokens at the last three positions; every call
    checks that the positions before it hold what was fed (a stale or
    missing row changes the result or fails)."""

    V = 7

    def __init__(self):
        self.cache: dict[int, int] = {}
        self.batches = 0

    def _logits(self, pos):
        for p in range(pos):
            assert p in self.cache, p
        x = [self.cache.get(pos - i, 0) for i in range(3)]
        nxt = (3 * x[0] + 2 * x[1] + x[2] + pos // 5) % self.V
        return -np.abs(np.arange(self.V, dtype=np.float32) - nxt)

    def prefill(self, toks, start, mode):
        for i, t in enumerate(toks):
            self.cache[start + i] = int(t)
        return self._logits(start + len(toks) - 1)

    def decode_step(self, tok, pos):
        self.cache[pos] = int(tok)
        for p in [q for q in self.cache if q > pos]:
            del self.cache[p]  # rows past pos were rejected drafts
        return self._logits(pos)

    def decode_step_batch(self, toks, start):
        assert 1 <= len(toks) <= 8
        self.batches += 1
        rows = []
        for i, t in enumerate(toks):
            self.cache[start + i] = int(t)
            rows.append(self._logits(start + i))
        return np.stack(rows)


@pytest.mark.parametrize("draft_len", [1, 2, 4, 8])
def test_speculative_equals_plain_on_toy_model(rt, draft_len):
    prompt = [1, 2, 3, 1, 2, 4, 1, 2, 3]
    plain, s0 = rt.generate_greedy(ToyCtx(), prompt, 60, draft_len=0, eos=())
    ctx = ToyCtx()
    spec, s1 = rt.generate_greedy(ctx, prompt, 60, draft_len=draft_len, eos=())
    assert spec == plain
    assert len(plain) == 60 and s0["spec_attempts"] == 0 and s0["decode_steps"] == 59
    assert s1["spec_attempts"] == ctx.batches > 0
    assert s1["spec_accepted"] + s1["decode_steps"] == 59


def test_generation_stops_at_eos_and_max_new(rt):
    prompt = [1, 2, 3, 1, 2, 4, 1, 2, 3]
    plain, _ = rt.generate_greedy(ToyCtx(), prompt, 60, draft_len=0, eos=())
    stop = plain[5]
    for draft_len in (0, 4):
        out, _ = rt.generate_greedy(ToyCtx(), prompt, 60, draft_len=draft_len, eos=(stop,))
        assert out[:6] == plain[:6] and out[-1] == stop
        if draft_len == 0:
            assert len(out) == 6
    for n in (1, 2, 7):
        out, _ = rt.generate_greedy(ToyCtx(), prompt, n, draft_len=4, eos=())
        assert out == plain[:n]


class OracleCtx:
    """The C oracle's Gemma-3 forward as a decode context (test infrastructure)."""

    def __init__(self, orc, cfg, layers, embed, fnorm):
        self.orc, self.cfg, self.layers, self.embed, self.fnorm = orc, cfg, copy.deepcopy(layers), embed, fnorm

    def prefill(self, toks, start, mode):
        return self.orc.gemma3_prefill(self.cfg, self.layers, self.embed, self.fnorm, toks, start, mode)

    def decode_step(self, tok, pos):
        return self.orc.gemma3_decode_step(self.cfg, self.layers, self.embed, self.fnorm, token=tok, pos=pos)

    def decode_step_batch(self, toks, start):
        return np.stack([self.decode_step(t, start + i) for i, t in enumerate(toks)])


# a prompt whose bigram (127, 127) is followed by other tokens: once the
# seed-0 tiny model settles on 127 the drafter proposes them and the verify
# rejects them (found on the oracle: 13 batches, 44 drafted, 38 kept)
SPEC_PROMPT = [11, 12, 13, 14, 11, 12, 13, 14, 127, 127, 5, 6, 7, 8]


def test_speculative_equals_plain_on_oracle_model(rt, orc):
    cfg = tiny(2)
    layers, embed, fnorm = make_model(orc, cfg, max_seq=64, ctx=0, seed=0)
    plain, _ = rt.generate_greedy(OracleCtx(orc, cfg, layers, embed, fnorm), SPEC_PROMPT, 40, draft_len=0)
    spec, st = rt.generate_greedy(OracleCtx(orc, cfg, layers, embed, fnorm), SPEC_PROMPT, 40, draft_len=4)
    assert spec == plain
    assert st["spec_attempts"] > 0 and st["spec_accepted"] < st["spec_drafted"]


@pytest.mark.gpu
def test_gpu_speculative_generation_matches_plain_and_oracle(rt, orc):
    """The batched verify in the loop: rejected drafts leave cache rows that
    the next call overwrites; the tokens equal plain greedy decoding on the
    GPU and on the oracle model."""
    cfg = tiny(2)
    max_seq = 64
    layers, embed, fnorm = make_model(orc, cfg, max_seq=max_seq, ctx=0, seed=0)
    ref, _ = rt.generate_greedy(OracleCtx(orc, cfg, layers, embed, fnorm), SPEC_PROMPT, 40, draft_len=0)
    runs = {}
    for draft_len in (0, 4):
        d = rt.HipDecodeContext(cfg, max_seq)
        for i, L in enumerate(layers):
            d.set_layer(i, L)
        d.set_embed(embed, fnorm)
        runs[draft_len] = rt.generate_greedy(d, SPEC_PROMPT, 40, draft_len=draft_len)
        d.close()
    (plain, s0), (spec, s1) = runs[0], runs[4]
    assert plain == ref
    assert spec == plain
    assert s0["decode_steps"] == 39
    assert s1["spec_attempts"] > 0 and s1["spec_accepted"] < s1["spec_drafted"]
