"""One generation request (dyllm/engine/sequence.py:8-82): prompt + ``max_new_tokens`` mask
tokens, unmasked block by block over the denoising steps."""
from __future__ import annotations

from enum import Enum, auto
from itertools import count
from typing import List

import numpy as np

from ..sampling_params import SamplingParams


class SequenceStatus(Enum):
    FULL = auto()
    SPARSE = auto()
    FINISHED = auto()


class Sequence:
    counter = count()

    def __init__(self, token_ids: List[int], sampling_params: SamplingParams = SamplingParams()):
        sp = sampling_params
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.FULL
        self.token_ids = list(token_ids)
        # int64 copy of token_ids for the per-step index building (update_token writes both)
        self.token_arr = np.asarray(self.token_ids, dtype=np.int64)
        self.mask_id = sp.mask_id
        # tokens written by the last step and their positions: the first layer's salient rows
        # of the next sparse step (model_runner.py:207-214)
        self.last_tokens = [self.token_ids[-1]] if self.token_ids else []
        self.last_token_pos = [0]
        self.output_length = sp.max_new_tokens
        self.num_full_steps = sp.num_full_steps
        self.num_steps = sp.steps
        self.processed_steps = 0
        self.num_prompt_tokens = sum(1 for t in self.token_ids if t != self.mask_id)
        self.num_tokens = self.num_prompt_tokens
        self.temperature = sp.temperature
        self.max_new_tokens = sp.max_new_tokens
        self.ignore_eos = sp.ignore_eos
        self.top_p = sp.top_p
        self.top_k = sp.top_k
        self.confidence_threshold = sp.confidence_threshold
        self.block_size = sp.block_size
        self.block_idx = 0

    def __len__(self):
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self) -> bool:
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return self.num_tokens - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> List[int]:
        return self.token_ids[: self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> List[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def answer_start(self) -> int:
        return len(self.token_ids) - self.max_new_tokens

    @property
    def num_transfer_tokens(self) -> int:
        """Tokens unmasked per step without a confidence threshold (sequence.py:68-71)."""
        if self.output_length % self.num_steps != 0:
            raise ValueError(f"max_new_tokens ({self.output_length}) must be a multiple of steps ({self.num_steps})")
        return self.output_length // self.num_steps

    def update_token(self, pos: List[int], token_id: List[int]):
        for p, t in zip(pos, token_id):
            if self.token_ids[p] == self.mask_id and t != self.mask_id:
                self.num_tokens += 1
            self.token_ids[p] = t
            self.token_arr[p] = t
        self.last_tokens = list(token_id)
        self.last_token_pos = list(pos)

    def update_block_idx(self):
        if self.num_completion_tokens > 0 and self.block_size > 0:
            self.block_idx = self.num_completion_tokens // self.block_size
