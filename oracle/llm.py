"""Oracle restatement of the CosyVoice3 LM head, speech embedding and a greedy decode.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows cv3cpu/models/llm.py:52-77,121 for the head and the embedding
gather.  The reference only samples (llm.py:112-149); greedy decoding here
is ``argmax`` of the head logits with ties to the lowest index, which is
what ``np.argsort(-p, kind="stable")[0]`` picks (llm.py:138), followed by
``speech_embedding[top]`` as the next input (llm.py:121).
"""

from __future__ import annotations

import numpy as np

from . import ops
from .qwen2 import Qwen2Config, Qwen2Model

SPEECH_TOKEN_SIZE = 6561   # llm.py:15


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
