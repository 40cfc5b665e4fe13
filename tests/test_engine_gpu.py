"""End-to-end engine on the GPU: continuous batching over a random-init Qwen3 of the 0.6B
geometry (2 layers, full vocabulary) against the CPU oracle forward pass.

Each generated token is checked teacher-forced: the oracle runs the whole final token list
of the sequence once, and the logit it gives the engine's token at that position must be
within LOGIT_TOL of the oracle's maximum (the two paths differ by bf16 rounding inside the
layers, so near-ties may legitimately flip), with >= 90% of the tokens equal to the
oracle's argmax. Prompts fit the token budget, so no prompt is chunked and token j of a
sequence is predicted at position prompt_len - 1 + j.
"""
import random
from types import SimpleNamespace

import pytest
import torch

import pagedkv.engine as E
from oracle import qwen3 as Q
from pagedkv.qwen3 import Qwen3Config

pytestmark = pytest.mark.gpu

LOGIT_TOL = 0.05   # absolute; the logits' spread over the vocabulary is ~0.6 here


def _cpu_weights(w):
    return SimpleNamespace(
        embed=w.embed.cpu(), final_norm=w.final_norm.cpu(),
        layers=[{k: v.cpu() for k, v in L.items()} for L in w.layers])


def _check(engine, cfg, prompts, outs):
    W = _cpu_weights(engine.runner.weights)
    total = agree = 0
    for p, out in zip(prompts, outs):
        logits = Q.forward_logits(W, cfg, p + out)
        for j, tok in enumerate(out):
            row = logits[len(p) - 1 + j]
            best = float(row.max())
            assert float(row[tok]) >= best - LOGIT_TOL, (j, tok, float(row[tok]), best)
            agree += int(int(row.argmax()) == tok)
            total += 1
    assert agree >= 0.9 * total, f"{agree}/{total} tokens equal the oracle argmax"


@pytest.mark.parametrize("eager", [False, True])
def test_engine_matches_oracle_teacher_forced(gpu, eager):
    cfg = Qwen3Config(num_hidden_layers=2)
    eng = E.LLMEngine(cfg, device=gpu, num_blocks=64, max_live_seqs=8, max_seq_len=1024,
                      enforce_eager=eager)
    rng = random.Random(3)
    lens = [37, 120, 256, 300, 5, 511]
    prompts = [[rng.randrange(cfg.vocab_size) for _ in range(n)] for n in lens]
    max_tokens = [6, 9, 3, 12, 7, 5]
    outs, stats = eng.generate(prompts, max_tokens, ignore_eos=True)
    assert [len(o) for o in outs] == max_tokens
    assert stats.output_tokens == sum(max_tokens)
    assert stats.decode_steps > 0 and stats.prefill_steps > 0
    _check(eng, cfg, prompts, outs)


def test_engine_graph_padding_and_block_crossing(gpu):
    # 3 live sequences replay the 4-wide graph (one padded row); contexts cross the
    # 256-token block boundary while decoding
    cfg = Qwen3Config(num_hidden_layers=2)
    eng = E.LLMEngine(cfg, device=gpu, num_blocks=32, max_live_seqs=4, max_seq_len=1024)
    rng = random.Random(4)
    prompts = [[rng.randrange(cfg.vocab_size) for _ in range(n)] for n in (250, 253, 100)]
    outs, stats = eng.generate(prompts, [10, 8, 4], ignore_eos=True)
    assert [len(o) for o in outs] == [10, 8, 4]
    assert eng.scheduler.num_free_blocks() == 32
    _check(eng, cfg, prompts, outs)


def test_engine_sizes_kv_cache_from_free_memory(gpu):
    """num_blocks None with gpu_memory_utilization: the cache takes what fits in that share
    of the device after the weights and the warmup forward's activations
    (model_runner.py:37-51,149-157), and the engine serves from it."""
    from pagedkv.runner import kv_cache_num_blocks

    cfg = Qwen3Config(num_hidden_layers=2)
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info(gpu)
    util = (total - free) / total + 0.03                  # about 3% of the device for the cache
    eng = E.LLMEngine(cfg, device=gpu, max_live_seqs=8, max_seq_len=1024, enforce_eager=True,
                      gpu_memory_utilization=util)
    # the warmup (16 prompts of 1024 tokens, the 16384-token budget) left its activation peak
    # above the weights for the sizing: at least the fused qkv output of those tokens
    assert eng.runner.activation_headroom >= 16384 * 4096 * 2
    nb = eng.runner.num_blocks
    block_bytes = 2 * cfg.num_hidden_layers * 256 * cfg.num_key_value_heads * cfg.head_dim * 2
    assert nb > 0 and nb * block_bytes <= total * util
    assert eng.runner.kv_cache.shape[2] == nb
    # nothing is left for a second cache of the same size at the same utilisation
    with pytest.raises(RuntimeError, match="Not enough GPU memory"):
        kv_cache_num_blocks(cfg.num_hidden_layers, 256, cfg.num_key_value_heads, cfg.head_dim, util,
                            requested=nb, device=gpu)
    rng = random.Random(4)
    prompts = [[rng.randrange(cfg.vocab_size) for _ in range(n)] for n in (40, 200)]
    outs, _ = eng.generate(prompts, [4, 6], ignore_eos=True)
    assert [len(o) for o in outs] == [4, 6]
