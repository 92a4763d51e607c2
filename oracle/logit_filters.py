"""CPU restatement of the decoding task's logit filters and greedy update
(TEST INFRASTRUCTURE ONLY: the tests compare the device-side filtered greedy
step against it; nothing in the product imports it).

Follows i_whisper/decoding.py statement by statement on float32 logits with
-inf masking:
  SuppressBlank.apply        decoding.py:426-433
  SuppressTokens.apply       decoding.py:436-441
  ApplyTimestampRules.apply  decoding.py:444-509
  GreedyDecoder.update       decoding.py:279-296 (temperature 0)
The filters run in the order DecodingTask builds them (decoding.py:556-572).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np


@dataclass
class FilterSpec:
    sample_begin: int                      # length of the initial tokens (prompt)
    eot: int
    suppress_tokens: List[int] = field(default_factory=list)
    blank_ids: Optional[List[int]] = None  # tokenizer.encode(" ") + [eot]; None = no SuppressBlank
    timestamp_begin: Optional[int] = None  # None = without_timestamps
    no_timestamps: Optional[int] = None
    max_initial_timestamp_index: Optional[int] = None


def _log_softmax(x: np.ndarray) -> np.ndarray:
    """float32 log_softmax along the last axis (x - max - log(sum(exp(x - max))))."""
    x = x.astype(np.float32)
    m = np.max(x, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, np.float32(0))
    e = np.exp(x - m, dtype=np.float32)
    return (x - m - np.log(np.sum(e, axis=-1, keepdims=True, dtype=np.float32))).astype(np.float32)


def _logsumexp(x: np.ndarray) -> np.float32:
    m = np.max(x)
    if not np.isfinite(m):
        return np.float32(m)
    return np.float32(m + np.log(np.sum(np.exp(x - m, dtype=np.float32), dtype=np.float32)))


def _masked(logits: np.ndarray, tokens: np.ndarray, spec: FilterSpec) -> np.ndarray:
    """Every filter step up to (not including) the final timestamp-probability rule."""
    logits = np.array(logits, dtype=np.float32, copy=True)
    L = tokens.shape[1]
    # SuppressBlank
    if spec.blank_ids is not None and L == spec.sample_begin:
        logits[:, spec.blank_ids] = -np.inf
    # SuppressTokens
    if spec.suppress_tokens:
        logits[:, spec.suppress_tokens] = -np.inf
    # ApplyTimestampRules, up to the probability rule
    tb = spec.timestamp_begin
    if tb is not None:
        if spec.no_timestamps is not None:
            logits[:, spec.no_timestamps] = -np.inf
        for k in range(tokens.shape[0]):
            sampled = tokens[k, spec.sample_begin:]
            seq = [int(t) for t in sampled]
            last_was_timestamp = len(seq) >= 1 and seq[-1] >= tb
            penultimate_was_timestamp = len(seq) < 2 or seq[-2] >= tb
            if last_was_timestamp:
                if penultimate_was_timestamp:
                    logits[k, tb:] = -np.inf
                else:
                    logits[k, :spec.eot] = -np.inf
            timestamps = sampled[sampled >= tb]
            if timestamps.size > 0:
                if last_was_timestamp and not penultimate_was_timestamp:
                    timestamp_last = int(timestamps[-1])
                else:
                    timestamp_last = int(timestamps[-1]) + 1
                logits[k, tb:timestamp_last] = -np.inf
        if L == spec.sample_begin:
            logits[:, :tb] = -np.inf
            if spec.max_initial_timestamp_index is not None:
                last_allowed = tb + spec.max_initial_timestamp_index
                logits[:, last_allowed + 1:] = -np.inf
    return logits


def apply_filters(logits: np.ndarray, tokens: np.ndarray, spec: FilterSpec) -> np.ndarray:
    """logits float32 [B, V] (a filtered copy is returned), tokens int64 [B, L]
    (prompt + sampled tokens)."""
    logits = _masked(logits, tokens, spec)
    tb = spec.timestamp_begin
    if tb is not None:
        # if sum of probability over timestamps is above any other token, sample timestamp
        logprobs = _log_softmax(logits)
        for k in range(tokens.shape[0]):
            timestamp_logprob = _logsumexp(logprobs[k, tb:])
            max_text_token_logprob = np.max(logprobs[k, :tb])
            if timestamp_logprob > max_text_token_logprob:
                logits[k, :tb] = -np.inf
    return logits


def greedy_next(logits: np.ndarray, tokens: np.ndarray, spec: FilterSpec) -> np.ndarray:
    """Next tokens [B] of GreedyDecoder.update after the filters."""
    f = apply_filters(logits, tokens, spec)
    nxt = np.argmax(f, axis=-1).astype(np.int64)  # first index of the maximum; 0 when all -inf
    nxt[tokens[:, -1] == spec.eot] = spec.eot
    return nxt


def timestamp_margin(logits: np.ndarray, tokens: np.ndarray, spec: FilterSpec) -> np.ndarray:
    """Per row |logsumexp over the allowed timestamps - the best allowed text
    logit| in float64 (inf where one side is empty): rows whose margin is at
    the level of fp32 rounding can flip the probability rule either way."""
    out = np.full(logits.shape[0], np.inf)
    if spec.timestamp_begin is None:
        return out
    tb = spec.timestamp_begin
    g = _masked(logits, tokens, spec).astype(np.float64)
    for k in range(g.shape[0]):
        ts, tx = g[k, tb:], g[k, :tb]
        ts = ts[np.isfinite(ts)]
        tx = tx[np.isfinite(tx)]
        if ts.size and tx.size:
            out[k] = abs(ts.max() + np.log(np.sum(np.exp(ts - ts.max()))) - tx.max())
    return out


def greedy_update(logits: np.ndarray, tokens: np.ndarray, eot: int, sum_logprobs: np.ndarray):
    """GreedyDecoder.update (decoding.py:279-296) at temperature 0 on float32
    logits [B, V] that the filters have already masked: returns the next tokens
    (EOT after EOT), the updated float32 sum of log-probabilities and whether
    every row's new token is EOT."""
    logits = np.asarray(logits, dtype=np.float32)
    nxt = np.argmax(logits, axis=-1).astype(np.int64)
    with np.errstate(invalid="ignore", divide="ignore"):
        current = _log_softmax(logits)[np.arange(logits.shape[0]), nxt]
        keep = (tokens[:, -1] != eot).astype(np.float32)
        sum_logprobs = (np.asarray(sum_logprobs, np.float32) + current * keep).astype(np.float32)
    nxt[tokens[:, -1] == eot] = eot
    return nxt, sum_logprobs, bool((nxt == eot).all())


def token_prob(logits: np.ndarray, token: int) -> np.ndarray:
    """softmax(logits.float())[:, token] (decoding.py:690-695), float32."""
    x = np.asarray(logits, dtype=np.float32)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m, dtype=np.float32)
    return (e[:, token] / np.sum(e, axis=-1, dtype=np.float32)).astype(np.float32)
