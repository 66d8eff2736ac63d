"""Oracle restatement of the CosyVoice3 LM head, speech embedding, sampler and decode loops.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/models/llm.py:52-77,121 for the head and the embedding
gather, llm.py:37-49 (nucleus_sampling) and llm.py:125-149 (_sample) for the
sampler, and llm.py:104-123 for the token loop.  Greedy decoding is ``argmax``
of the head logits with ties to the lowest index, which is what
``np.argsort(-p, kind="stable")[0]`` picks (llm.py:138), followed by
``speech_embedding[top]`` as the next input (llm.py:121).
"""

from __future__ import annotations

import numpy as np

from . import ops
from .qwen2 import Qwen2Config, Qwen2Model

SPEECH_TOKEN_SIZE = 6561   # llm.py:15


class Sampling:
    """The SamplingConfig fields the sampler reads (llm.py:18-34)."""

    def __init__(self, top_p=0.8, top_k=25, win_size=10, tau_r=0.1, seed=None, strict_min_len=False):
        self.top_p, self.top_k, self.win_size, self.tau_r = top_p, top_k, win_size, tau_r
        self.strict_min_len = strict_min_len
        self.rng = np.random.default_rng(seed)


def nucleus_sampling(probs_sorted, idx_sorted, rng, top_p, top_k):
    """Entries in order until their float64 running sum reaches top_p, at most top_k, then
    one draw from them renormalised (llm.py:37-49)."""
    cum = 0.0
    n = 0
    for i in range(min(top_k, idx_sorted.shape[0])):
        if cum >= top_p:
            break
        cum += float(probs_sorted[i])
        n += 1
    p = probs_sorted[:n].astype(np.float64)
    p = p / p.sum()
    return int(idx_sorted[rng.choice(n, p=p)])


def sample(logp, decoded, cfg, ignore_eos: bool, strict_min_len: bool, speech_token_size: int) -> int:
    """llm.py:125-149: mask eos below min_len, stable descending order, nucleus draw,
    then a draw from the full distribution without the pick when the pick fills
    win_size * tau_r of the recent window."""
    scores = logp.copy()
    if ignore_eos:
        if strict_min_len:
            scores[speech_token_size:speech_token_size + 200] = -np.inf
        else:
            scores[speech_token_size] = -np.inf
    probs = ops.softmax(scores)
    order = np.argsort(-probs, kind="stable")
    top = nucleus_sampling(probs[order], order, cfg.rng, cfg.top_p, cfg.top_k)
    window = decoded[-cfg.win_size:]
    rep = sum(1 for t in window if t == top)
    if rep >= cfg.win_size * cfg.tau_r:
        scores[top] = -np.inf
        p = ops.softmax(scores).astype(np.float64)
        p /= p.sum()
        top = int(cfg.rng.choice(p.shape[0], p=p))
    return top


class CosyVoice3LM:
    def __init__(self, weights, prefix: str = "llm."):
        self.w = weights
        self.prefix = prefix
        self.cfg = Qwen2Config.from_meta(weights.meta)
        self.body = Qwen2Model(weights, self.cfg, prefix=prefix + "model.")
        self.speech_token_size = int(weights.meta.get("speech_token_size", SPEECH_TOKEN_SIZE))
        self.sos = self.speech_token_size + 0
        self.task_id = self.speech_token_size + 2

    def speech_emb(self, ids):
        """llm.py:68-69"""
        return ops.embedding(self.w.get(self.prefix + "speech_embedding"), np.asarray(ids))

    def text_emb(self, ids):
        """llm.py:71-72"""
        return self.body.embed(np.asarray(ids))

    def head(self, h):
        """llm_decoder linear, optional bias (llm.py:74-77)."""
        name = self.prefix + "llm_decoder.bias"
        bias = self.w.get(name) if name in self.w else None
        return ops.linear(h, self.w.get(self.prefix + "llm_decoder.weight"), bias)

    def sample(self, logp, decoded, cfg, ignore_eos: bool, strict_min_len: bool) -> int:
        """llm.py:125-149"""
        return sample(logp, decoded, cfg, ignore_eos, strict_min_len, self.speech_token_size)

    def sampled(self, first_input, cache, max_len: int, min_len: int, cfg):
        """The token loop of generate() (llm.py:104-123) from its first input: log_softmax of
        the head logits, sample, stop on any of the 200 control ids."""
        x = first_input
        out = []
        stop = range(self.speech_token_size, self.speech_token_size + 200)
        for i in range(max_len):
            logits = self.head(self.body.forward(x, cache)[-1:]).astype(np.float32)
            logp = ops.log_softmax(logits, axis=-1)[0]
            top = self.sample(logp, out, cfg, i < min_len, cfg.strict_min_len)
            if top in stop:
                break
            out.append(top)
            x = self.speech_emb([top])
        return out

    def greedy(self, first_input, cache, steps: int):
        """Greedy tokens: argmax(head(body(x)[-1])), next input speech_emb[top]."""
        x = first_input
        out = []
        for _ in range(steps):
            logits = self.head(self.body.forward(x, cache)[-1:])[0]
            top = int(np.argmax(logits))
            out.append(top)
            x = self.speech_emb([top])
        return out
