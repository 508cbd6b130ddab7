"""Chat: the `chat` command's rolling context (src/LLM.Cli/Program.cs:736-768) on a HIP session.

The history starts as [eos]; each turn appends the user's ids, keeps the last
2 x ContextLength ids, and streams Sampler.Generate over the whole history
(which itself left-truncates to the window) with the turn's eos, appending every
id it yields.  One Random (seed) is shared by all turns, one NextDouble per
sampled step.  /reset is ``reset()``.  Tokenizer encode/decode stay with the
caller (the reference's BpeTokenizer and Utf8StreamDecoder).
"""
from __future__ import annotations

from typing import Iterator, Sequence

from .model import GptModel, Random
from .sampler import Sampler


class Chat:
    def __init__(self, model: GptModel, eos_id: int, tokens_per_turn: int = 100, temperature: float = 0.8,
                 top_k: int = 40, repetition_penalty: float = 1.0, no_repeat_ngram: int = 0, seed: int = 1,
                 chunk: int = 16):
        self.model = model
        self.eos_id = int(eos_id)
        self.tokens_per_turn = int(tokens_per_turn)
        self.temperature = float(temperature)
        self.top_k = int(top_k)
        self.repetition_penalty = float(repetition_penalty)
        self.no_repeat_ngram = int(no_repeat_ngram)
        self.rng = Random(seed)
        self.chunk = int(chunk)
        self.history = [self.eos_id]

    def reset(self) -> None:
        """/reset: the context back to [eos]."""
        self.history = [self.eos_id]

    def turn(self, user_ids: Sequence[int]) -> Iterator[int]:
        """One exchange: yields the model's ids as they are generated (an empty line
        just lets the model continue)."""
        self.history.extend(int(t) for t in user_ids)
        keep = self.model.config.context_length * 2
        if len(self.history) > keep:
            del self.history[:len(self.history) - keep]
        for tid in Sampler.generate_stream(self.model, self.history, self.tokens_per_turn, self.temperature,
                                           self.top_k, self.rng, eos_id=self.eos_id,
                                           repetition_penalty=self.repetition_penalty,
                                           no_repeat_ngram_size=self.no_repeat_ngram, chunk=self.chunk):
            self.history.append(tid)
            yield tid
