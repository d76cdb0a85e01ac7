"""Generation engine (dyllm/engine/llm_engine.py:23-312): requests in, a step loop of
schedule -> run -> postprocess, decoded texts out. One process drives the one GPU."""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Union

from ..config import CONFIG_FIELDS, Config
from ..sampling_params import SamplingParams
from ..utils.metadata import get_metadata, reset_metadata
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import Sequence


def load_tokenizer(model_dir: Optional[str]):
    """The checkpoint's tokenizer when the model directory holds one, else None (token-id
    prompts only). No code from the directory is executed."""
    if model_dir is None:
        return None
    names = ("tokenizer.json", "tokenizer_config.json", "tokenizer.model", "vocab.json")
    if not any(os.path.isfile(os.path.join(model_dir, n)) for n in names):
        return None
    from transformers import AutoTokenizer

    return AutoTokenizer.from_pretrained(model_dir, use_fast=True, trust_remote_code=False, local_files_only=True)


class DLLMEngine:

    def __init__(self, model: str, threshold: float = 0.99, model_runner: Optional[ModelRunner] = None, **kwargs):
        unknown = set(kwargs) - CONFIG_FIELDS
        if unknown:
            raise TypeError(f"unknown engine options {sorted(unknown)}")
        config = Config(model, threshold=threshold, **kwargs)
        self.config = config
        os.environ.setdefault("TOKENIZERS_PARALLELISM", "false")
        self.tokenizer = load_tokenizer(config.model_dir)
        if self.tokenizer is not None and self.tokenizer.eos_token_id is not None:
            config.eos = self.tokenizer.eos_token_id
        self.mask = config.mask_id
        reset_metadata()
        self.model_runner = model_runner if model_runner is not None else ModelRunner(config)
        self.scheduler = Scheduler(config)
        self._closed = False

    # -- requests -------------------------------------------------------------------------
    def _create_sequence(self, prompt: Union[str, List[int]], sp: SamplingParams) -> Sequence:
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("this model has no tokenizer files: pass prompts as token-id lists")
            token_ids = self.tokenizer.encode(prompt)
        else:
            token_ids = [int(t) for t in prompt]
        if sp.input_len is not None:
            if not token_ids:
                raise ValueError("input_len cannot be applied to an empty prompt")
            token_ids = token_ids[: sp.input_len] + [token_ids[-1]] * max(0, sp.input_len - len(token_ids))
        if self.mask is not None:
            token_ids = token_ids + [self.mask] * sp.max_new_tokens
        if len(token_ids) > self.config.max_model_len:
            raise ValueError(f"prompt + max_new_tokens = {len(token_ids)} exceeds max_model_len "
                             f"{self.config.max_model_len}")
        sp.mask_id = self.mask
        return Sequence(token_ids, sp)

    def add_request(self, prompt: Union[str, List[int]], sampling_params: SamplingParams) -> int:
        seq = self._create_sequence(prompt, sampling_params)
        self.scheduler.add(seq)
        return seq.seq_id

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    @property
    def execution_stats(self) -> Dict[str, int]:
        return {"full_forwards": self.model_runner.num_full_forwards,
                "sparse_forwards": self.model_runner.num_sparse_forwards}

    def step(self):
        seqs, is_full = self.scheduler.schedule()
        finished_prev = list(get_metadata().finished_seqs)
        pos, tok, cnt = self.model_runner.call("run", seqs, is_full, finished_prev)
        self.scheduler.postprocess(seqs, pos, tok, cnt)
        outputs = [(s.seq_id, s.token_ids) for s in seqs if s.is_finished]
        num_tokens = sum(len(s) for s in seqs) if is_full else -len(seqs)
        return outputs, num_tokens

    def _decode(self, ids: List[int]) -> str:
        if self.tokenizer is None:
            return ""
        return self.tokenizer.decode(ids, skip_special_tokens=True)

    def generate(self, prompts: Union[List[str], List[List[int]]],
                 sampling_params: Union[SamplingParams, List[SamplingParams]]) -> List[dict]:
        """-> [{"text", "token_ids"}] in request order (llm_engine.py:267-297); ``text`` decodes
        the ``max_new_tokens`` answer tokens, ``token_ids`` is the whole sequence."""
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        if len(sampling_params) != len(prompts):
            raise ValueError("one SamplingParams per prompt, or a single one for all")
        order = []
        for prompt, sp in zip(prompts, sampling_params):
            order.append((self.add_request(prompt, SamplingParams(**vars(sp))), sp.max_new_tokens))
        done: Dict[int, List[int]] = {}
        while not self.is_finished():
            out, _ = self.step()
            for sid, ids in out:
                done[sid] = ids
        return [{"text": self._decode(done[sid][-n:] if n > 0 else []), "token_ids": done[sid]} for sid, n in order]

    def exit(self):
        if not self._closed:
            self.model_runner.call("exit")
            self._closed = True
