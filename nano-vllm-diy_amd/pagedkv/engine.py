"""Offline continuous-batching engine over the host core and the model runner.

Mirrors LLMEngine (src/engine/llm_engine.py): add_request with the reference's capacity
checks (:70-105), step = schedule -> run -> postprocess (:107-112), generate over token-id
prompts (:116-148). Sampling is greedy (the serving benchmark's setting); the reference's
tokenizer and tensor-parallel workers are not part of this engine.
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from ._host import HostScheduler
from .qwen3 import Qwen3Config
from .runner import ModelRunner


@dataclass
class GenerateStats:
    wall_s: float
    steps: int
    prefill_steps: int
    decode_steps: int
    prefill_tokens: int
    decode_tokens: int
    output_tokens: int

    @property
    def tok_per_s(self) -> float:
        return self.output_tokens / self.wall_s if self.wall_s > 0 else 0.0


class LLMEngine:
    def __init__(self, cfg: Qwen3Config = Qwen3Config(), device: str | torch.device = "cuda",
                 num_blocks: int | None = None, block_size: int = 256, max_num_seqs: int = 512,
                 max_num_batched_tokens: int = 16384, chunked_prefill_size: int = 512,
                 max_live_seqs: int = 128, max_seq_len: int = 8192, enforce_eager: bool = False,
                 eos: int = 151645, seed: int = 5, gpu_memory_utilization: float | None = None):
        """num_blocks None: with gpu_memory_utilization, as many blocks as fit in that share of
        the device (the reference's sizing, model_runner.py:149-157); without it, enough for
        max_live_seqs sequences of max_seq_len tokens."""
        # RunnerConfig caps the model's context at 8192 (runner_config.py:13,41)
        self.max_seq_len = min(max_seq_len, cfg.max_position_embeddings)
        if num_blocks is None and gpu_memory_utilization is None:
            num_blocks = max_live_seqs * ((self.max_seq_len + block_size - 1) // block_size)
        self.runner = ModelRunner(cfg, device, num_blocks, block_size, self.max_seq_len,
                                  min(max_num_seqs, max_live_seqs, 512), enforce_eager, seed,
                                  gpu_memory_utilization or 0.9, max_num_batched_tokens, max_num_seqs)
        num_blocks = self.runner.num_blocks
        self.scheduler = HostScheduler(num_blocks, block_size, max_num_seqs, max_num_batched_tokens,
                                       chunked_prefill_size, max_live_seqs, eos, self.max_seq_len)

    def add_request(self, prompt: list[int], max_tokens: int, ignore_eos: bool = False) -> int:
        if len(prompt) + max_tokens > self.max_seq_len:          # llm_engine.py:98-102
            raise ValueError(f"prompt {len(prompt)} + max_tokens {max_tokens} exceeds the "
                             f"maximum sequence length {self.max_seq_len}")
        return self.scheduler.add_request(prompt, max_tokens, ignore_eos)

    def step(self):
        """One engine step; returns (step, number of sequences that finished) or None."""
        st = self.scheduler.schedule()
        if st is None:
            return None
        toks = self.runner.run(st)
        return st, self.scheduler.postprocess(toks)

    def generate(self, prompts: list[list[int]], max_tokens: int | list[int],
                 ignore_eos: bool = False) -> tuple[list[list[int]], GenerateStats]:
        if not isinstance(max_tokens, list):
            max_tokens = [max_tokens] * len(prompts)
        t0 = time.perf_counter()
        ids = [self.add_request(p, m, ignore_eos) for p, m in zip(prompts, max_tokens)]
        steps = pf_steps = dec_steps = pf_tok = dec_tok = 0
        while True:
            res = self.step()
            if res is None:
                break
            st, _ = res
            steps += 1
            pf_tok += st.num_prefill_tokens
            dec_tok += st.num_decode_tokens
            if st.is_prefill:
                pf_steps += 1
            else:
                dec_steps += 1
        outs = [self.scheduler.generated(i) for i in ids]
        wall = time.perf_counter() - t0
        stats = GenerateStats(wall, steps, pf_steps, dec_steps, pf_tok, dec_tok,
                              sum(len(o) for o in outs))
        return outs, stats
