"""Model runner: KV cache, eager prefill steps and HIP-graph decode steps.

Mirrors ModelRunner (src/engine/model_runner.py): the KV cache is one tensor
(2, layers, blocks, block_size, Hkv, D) with per-layer views (:138-166); a step with more
than one query row in some sequence runs eagerly (:242-243); a decode step with at most
the largest captured batch replays the graph of the next captured size, with the
reference's padding -- slot -1, zeroed cu_seqlens tail, -1 block tables (:244-259) -- and
graphs are captured from the largest size down with one shared memory pool (:268-315).

Differences by design: the greedy LM head runs inside the decode graph (the reference
computes logits after the replay and samples outside); graphs are captured per batch size
AND per context bucket (max_seqlen_k rounded up to a power of two from 512 to
max_seq_len), because the decode kernel sizes its key splits from max_seqlen_k -- one
graph at max_seq_len would give a batch of short contexts a few long splits and leave most
of the GPU idle; and the padded decode inputs are staged in two packed pinned host
buffers whose device twins hold the graphs' static inputs, so a decode step is two
host-to-device copies and one graph launch.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from ._host import Step
from .context import Context
from .qwen3 import Qwen3Config, Qwen3Model, Qwen3Weights


def graph_batch_sizes(max_bs: int) -> list[int]:
    """Captured decode batch sizes: 1, 2, 4, 8, then multiples of 16 (model_runner.py:284)."""
    return [b for b in (1, 2, 4, 8) if b <= max_bs] + list(range(16, max_bs + 1, 16))


def context_buckets(max_seq_len: int, smallest: int = 512) -> list[int]:
    """max_seqlen_k values the decode graphs are captured for: powers of two, then the cap."""
    out, b = [], smallest
    while b < max_seq_len:
        out.append(b)
        b *= 2
    return out + [max_seq_len]


def kv_cache_num_blocks(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int,
                        gpu_memory_utilization: float = 0.9, requested: int | None = None,
                        itemsize: int = 2, device: torch.device | str | None = None) -> int:
    """KV-cache blocks that fit in gpu_memory_utilization of the device, as the reference
    sizes its cache (model_runner.py:149-157): total x utilization, minus what is in use,
    minus the allocator's peak beyond its current allocation (the activations a forward pass
    needs on top of the weights), divided by one block's K and V over all layers. A request
    above that raises, as the reference's assert does; requested None or <= 0 takes them all.
    """
    free, total = torch.cuda.mem_get_info(device)
    used = total - free
    stats = torch.cuda.memory_stats(device)
    peak = stats["allocated_bytes.all.peak"]
    current = stats["allocated_bytes.all.current"]
    block_bytes = 2 * num_layers * block_size * num_kv_heads * head_dim * itemsize
    max_blocks = int(total * gpu_memory_utilization - used - peak + current) // block_bytes
    if requested is None or requested <= 0:
        requested = max_blocks
    if requested > max_blocks:
        raise RuntimeError(f"Not enough GPU memory to allocate kv cache, required "
                           f"{requested * block_bytes / 2**30:.2f} GB but only "
                           f"{max_blocks * block_bytes / 2**30:.2f} GB is available")
    return requested


class ModelRunner:
    def __init__(self, cfg: Qwen3Config, device: torch.device | str, num_blocks: int | None,
                 block_size: int = 256, max_seq_len: int = 8192, max_graph_bs: int = 128,
                 enforce_eager: bool = False, seed: int = 5, gpu_memory_utilization: float = 0.9,
                 max_num_batched_tokens: int = 16384, max_num_seqs: int = 512):
        """As the reference's runner (model_runner.py:35-56): the weights, a warmup forward at
        the largest step (warmup_model), then the KV cache -- num_blocks None: as many blocks
        as fit in gpu_memory_utilization of the device beside the weights and the warmup's
        activation peak (kv_cache_num_blocks) -- then the decode graphs."""
        self.cfg = cfg
        self.dev = torch.device(device)
        self.block_size = block_size
        self.max_seq_len = max_seq_len
        L, Hkv, D = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
        self.weights = Qwen3Weights(cfg, self.dev, seed)
        self.model = Qwen3Model(cfg, self.weights, None, None, cfg.max_position_embeddings)
        self.warmup_model(max_num_batched_tokens, max_seq_len, max_num_seqs)
        stats = torch.cuda.memory_stats(self.dev)
        # what the sizing keeps free for activations: the warmup's peak above the weights
        self.activation_headroom = stats["allocated_bytes.all.peak"] - stats["allocated_bytes.all.current"]
        if num_blocks is None:
            num_blocks = kv_cache_num_blocks(L, block_size, Hkv, D, gpu_memory_utilization, device=self.dev)
        self.num_blocks = num_blocks
        self.kv_cache = torch.empty(2, L, num_blocks, block_size, Hkv, D, dtype=torch.bfloat16,
                                    device=self.dev)
        self.model.bind_caches(self.kv_cache[0], self.kv_cache[1])
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self.graph_bs: list[int] = []
        self.buckets: list[int] = []
        if not enforce_eager and max_graph_bs > 0:
            self._capture(max_graph_bs)

    def warmup_model(self, max_num_batched_tokens: int, max_seq_len: int, max_num_seqs: int) -> None:
        """The reference's warmup_model (model_runner.py:116-129): free the allocator's cache,
        reset its peak, run one prefill of min(budget, max_seq_len)-token sequences of token 0
        filling the token budget (no KV cache yet: dense attention over the fresh keys, no
        store), and free the cache again, so the peak records a forward pass's activations
        above the weights. It also loads every library kernel the prefill path uses before the
        cache is sized."""
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(self.dev)
        seq_len = min(max_num_batched_tokens, max_seq_len)
        num_seqs = max(1, min(max_num_batched_tokens // seq_len, max_num_seqs))
        n = seq_len * num_seqs
        cu = torch.arange(0, n + 1, seq_len, dtype=torch.int32, device=self.dev)
        ctx = Context(is_prefill=True, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=seq_len,
                      max_seqlen_k=seq_len, slot_mapping=None, context_lens=None, block_tables=None)
        ids = torch.zeros(n, dtype=torch.int64, device=self.dev)
        pos = torch.arange(seq_len, dtype=torch.int64, device=self.dev).repeat(num_seqs)
        hidden = self.model.forward(ids, pos, ctx)
        self.model.greedy(hidden, ctx)
        torch.cuda.synchronize(self.dev)
        del hidden
        torch.cuda.empty_cache()

    # ------------------------------------------------------------------ eager ----
    def _to_dev(self, t: torch.Tensor) -> torch.Tensor:
        return t.to(self.dev, non_blocking=True)

    def run_eager(self, step: Step) -> torch.Tensor:
        ctx = Context(is_prefill=step.is_prefill, cu_seqlens_q=self._to_dev(step.cu_seqlens_q),
                      cu_seqlens_k=self._to_dev(step.cu_seqlens_k), max_seqlen_q=step.max_seqlen_q,
                      max_seqlen_k=step.max_seqlen_k, slot_mapping=self._to_dev(step.slot_mapping),
                      context_lens=None,
                      block_tables=None if step.block_tables is None else self._to_dev(step.block_tables))
        hidden = self.model.forward(self._to_dev(step.input_ids), self._to_dev(step.positions), ctx)
        return self.model.greedy(hidden, ctx)

    # ------------------------------------------------------------------ graphs ---
    def _capture(self, max_bs: int) -> None:
        self.max_blocks = (self.max_seq_len + self.block_size - 1) // self.block_size
        mb = self.max_blocks
        # packed staging: int64 [ids | positions], int32 [cu_q | cu_k | slots | block tables]
        self.n64 = 2 * max_bs
        self.n32 = 2 * (max_bs + 1) + max_bs + max_bs * mb
        pin = dict(pin_memory=True)
        self.h64 = torch.zeros(self.n64, dtype=torch.int64, **pin)
        self.h32 = torch.zeros(self.n32, dtype=torch.int32, **pin)
        self.d64 = torch.zeros(self.n64, dtype=torch.int64, device=self.dev)
        self.d32 = torch.zeros(self.n32, dtype=torch.int32, device=self.dev)
        self.np64, self.np32 = self.h64.numpy(), self.h32.numpy()
        o = np.cumsum([0, max_bs + 1, max_bs + 1, max_bs])
        self.off = dict(cu_q=int(o[0]), cu_k=int(o[1]), slots=int(o[2]), bt=int(o[3]))
        self.max_bs = max_bs
        d64, d32, off = self.d64, self.d32, self.off
        ids, pos = d64[:max_bs], d64[max_bs:]
        cu_q = d32[off["cu_q"]:off["cu_q"] + max_bs + 1]
        cu_k = d32[off["cu_k"]:off["cu_k"] + max_bs + 1]
        slots = d32[off["slots"]:off["slots"] + max_bs]
        bt = d32[off["bt"]:].view(max_bs, mb)
        slots.fill_(-1)
        bt.fill_(-1)
        self.np32[off["slots"]:off["slots"] + max_bs] = -1
        self.np32[off["bt"]:] = -1
        self.tokens = torch.zeros(max_bs, dtype=torch.int32, device=self.dev)
        self.graph_bs = graph_batch_sizes(max_bs)
        self.buckets = context_buckets(self.max_seq_len)
        # buffers the kernels reuse inside the graphs, sized for the largest batch up front
        ops.reserve_workspace(max_bs, self.cfg.num_attention_heads, self.cfg.head_dim, 1,
                              self.max_seq_len, self.dev)
        ops.reserve_linear_workspace(self.model.linear_workspace_bytes(max_bs), self.dev)
        ops.lm_head_greedy(torch.zeros(max_bs, self.cfg.hidden_size, dtype=torch.bfloat16,
                                       device=self.dev), self.weights.embed)
        pool = None
        for bs in reversed(self.graph_bs):
            for kb in reversed(self.buckets):
                ctx = Context(is_prefill=False, cu_seqlens_q=cu_q[:bs + 1],
                              cu_seqlens_k=cu_k[:bs + 1], max_seqlen_q=1, max_seqlen_k=kb,
                              slot_mapping=slots[:bs], context_lens=None, block_tables=bt[:bs])
                hidden = self.model.forward(ids[:bs], pos[:bs], ctx)            # warmup
                self.model.greedy(hidden, ctx, out=self.tokens[:bs])
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool):
                    hidden = self.model.forward(ids[:bs], pos[:bs], ctx)
                    self.model.greedy(hidden, ctx, out=self.tokens[:bs])
                if pool is None:
                    pool = g.pool()
                self.graphs[(bs, kb)] = g
        torch.cuda.synchronize()

    def run_graph(self, step: Step) -> torch.Tensor:
        S = step.num_seqs
        bs = next(b for b in self.graph_bs if b >= S)
        mb, off = self.max_blocks, self.off
        n64, n32 = self.np64, self.np32
        n64[:S] = step.input_ids.numpy()
        n64[self.max_bs:self.max_bs + S] = step.positions.numpy()
        cq = off["cu_q"]
        n32[cq:cq + S + 1] = step.cu_seqlens_q.numpy()
        n32[cq + S + 1:cq + bs + 1] = 0
        ck = off["cu_k"]
        n32[ck:ck + S + 1] = step.cu_seqlens_k.numpy()
        n32[ck + S + 1:ck + bs + 1] = 0
        sl = off["slots"]
        n32[sl:sl + S] = step.slot_mapping.numpy()
        n32[sl + S:sl + bs] = -1
        bt = n32[off["bt"]:].reshape(self.max_bs, mb)
        w = step.block_tables.shape[1]
        bt[:bs, :] = -1
        bt[:S, :w] = step.block_tables.numpy()
        self.d64.copy_(self.h64, non_blocking=True)
        self.d32[:off["bt"] + bs * mb].copy_(self.h32[:off["bt"] + bs * mb], non_blocking=True)
        kb = next(b for b in self.buckets if b >= step.max_seqlen_k)
        self.graphs[(bs, kb)].replay()
        return self.tokens[:S]

    # ------------------------------------------------------------------ step -----
    def run(self, step: Step) -> np.ndarray:
        """Greedy next token of every scheduled sequence (batch order), on the host."""
        use_graph = (not step.is_prefill and self.graphs and step.num_seqs <= self.graph_bs[-1]
                     and step.block_tables is not None and step.max_seqlen_k <= self.buckets[-1])
        toks = self.run_graph(step) if use_graph else self.run_eager(step)
        return toks.cpu().numpy()
