"""Greedy generation with n-gram speculative decoding over a decode context.

Host logic above the C ABI: the caller of `rt_decode_prefill`,
`rt_decode_step` and `rt_decode_step_batch` in the reference's generation
loop.  `generate_greedy` runs on any object with the three methods of
`HipDecodeContext` it uses (`prefill`, `decode_step`, `decode_step_batch`).
"""
from __future__ import annotations

import numpy as np

# Gemma 3's two end-of-sequence ids, <eos> and <end_of_turn> (transformer4.rs:2078)
GEMMA3_EOS = (1, 106)


class NgramDraftEngine:
    """NgramDraftEngine (transformer4.rs:1990-2032).

    draft(): for n = max_n down to 2, the last n tokens of the history are
    searched for from the start of the history (the suffix itself excluded);
    the first occurrence whose continuation is not empty returns up to
    max_draft tokens that followed it.  No match, or fewer than two tokens of
    history, drafts nothing."""

    def __init__(self, max_n: int, max_draft: int):
        self.history: list[int] = []
        self.max_n = max_n
        self.max_draft = max_draft

    def record(self, token: int) -> None:
        self.history.append(int(token))

    def record_many(self, tokens) -> None:
        self.history.extend(int(t) for t in tokens)

    def draft(self) -> list[int]:
        h, size = self.history, len(self.history)
        if size < 2:
            return []
        for n in range(min(self.max_n, size), 1, -1):
            suffix = h[size - n:]
            for start in range(size - n):
                if h[start:start + n] == suffix:
                    cont_start = start + n
                    cont_end = min(cont_start + self.max_draft, size)
                    if cont_start < cont_end:
                        return h[cont_start:cont_end]
        return []


def greedy_token(logits) -> int:
    """sample_token at temperature 0 with repetition penalty 1
    (transformer4.rs:2994-3092): the softmax probabilities in f32
    (exp(s - max), divided by their sum taken in index order) and the index of
    the largest, the last one among equals (Iterator::max_by)."""
    s = np.asarray(logits, dtype=np.float32).ravel()
    p = np.exp(s - s.max(), dtype=np.float32)
    total = np.add.accumulate(p, dtype=np.float32)[-1]
    p = (p / total).astype(np.float32)
    return int(p.size - 1 - int(np.argmax(p[::-1])))


def generate_greedy(ctx, prompt, max_new: int, draft_len: int = 0, eos=GEMMA3_EOS, prefill_mode: int = 0):
    """generate_cached_streaming's decode loop at temperature 0
    (transformer4.rs:2045-2430, the GPU branch): the prompt is prefilled and
    its last row gives the first token; each later step either verifies an
    n-gram draft in one batch (draft_len > 0 and a non-empty draft) or runs one
    decode step.

    Verify: with k = min(len(draft), max_new - step) the batch holds the
    previous token and draft[0 .. k-2] at positions seq_len, seq_len+1, ...;
    row i's greedy token is emitted, and the walk stops after the first one
    that differs from draft[i] (that token is emitted too).  seq_len advances
    by the tokens emitted: the cache rows written for rejected drafts are
    overwritten by the next call.  An end-of-sequence token ends the loop
    after the batch it came in (the reference checks the last token only).

    Returns (tokens, stats) with stats = {"spec_attempts", "spec_drafted",
    "spec_accepted", "decode_steps"}."""
    prompt = [int(t) for t in prompt]
    if not prompt:
        raise ValueError("generate_greedy: empty prompt")
    if max_new < 1:
        return [], {"spec_attempts": 0, "spec_drafted": 0, "spec_accepted": 0, "decode_steps": 0}
    ngram = NgramDraftEngine(4, draft_len)
    ngram.record_many(prompt)
    first = greedy_token(ctx.prefill(prompt, 0, prefill_mode))
    out = [first]
    ngram.record(first)
    stats = {"spec_attempts": 0, "spec_drafted": 0, "spec_accepted": 0, "decode_steps": 0}
    if first in eos:
        return out, stats
    seq_len, prev, step, hit_eos = len(prompt), first, 1, False
    while step < max_new and not hit_eos:
        did_speculate = False
        if draft_len > 0:
            draft = ngram.draft()
            if draft:
                k = min(len(draft), max_new - step)
                verify = [prev] + draft[:k - 1]
                rows = ctx.decode_step_batch(verify, seq_len)
                stats["spec_attempts"] += 1
                stats["spec_drafted"] += k
                accepted = 0
                for i in range(k):
                    tok = greedy_token(rows[i])
                    out.append(tok)
                    ngram.record(tok)
                    prev = tok
                    accepted += 1
                    if tok != draft[i]:
                        break
                stats["spec_accepted"] += accepted
                seq_len += accepted
                step += accepted
                hit_eos = prev in eos
                did_speculate = True
        if hit_eos:
            break
        if not did_speculate:
            logits = ctx.decode_step(prev, seq_len)
            seq_len += 1
            stats["decode_steps"] += 1
            prev = greedy_token(logits)
            out.append(prev)
            ngram.record(prev)
            step += 1
            hit_eos = prev in eos
    return out, stats
