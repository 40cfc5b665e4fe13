"""GPU parity of the serving loop's other kernels (residual RMSNorm, SiLU * mul, greedy LM
head) against the oracle, through the C-ABI.

Bars: norm and SiLU outputs within 1 bf16 ulp element-wise and identical on >= 99% of
elements (the reference runs them under torch.compile: FMA contraction and rsqrt are not
pinned). Greedy tokens: the chosen token's bf16 logit (fp64 dot product) within 1 ulp of
the row's maximum for every row, and the oracle's token (lowest id among equal bf16
maxima) on >= 97% of rows -- two ids whose fp32 logits straddle a bf16 rounding boundary
can legitimately swap.
"""
import pytest
import torch

import pagedkv
from oracle import model_ops as M
from oracle import producer as P
from test_oracle_producer import ulp_diff

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 151936, 1024


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _close(got, want, what):
    d = ulp_diff(got.cpu(), want.cpu())
    assert int(d.max()) <= 1, f"{what}: max ulp {int(d.max())}"
    assert float((d == 0).float().mean()) >= 0.99, what


@pytest.mark.parametrize("rows,hidden", [(37, 1024), (5, 2048), (3, 4096), (9, 520)])
def test_add_rmsnorm_matches_oracle(gpu, rows, hidden):
    x, r = _rand((rows, hidden), rows, 2.0), _rand((rows, hidden), rows + 1)
    w = (_rand((hidden,), 7, 0.3).float() + 1).to(torch.bfloat16)
    out = pagedkv.add_rmsnorm(x.to(gpu), w.to(gpu), 1e-6)
    _close(out, P.rms_norm(x, w, 1e-6), "normal")
    out, res = pagedkv.add_rmsnorm(x.to(gpu), w.to(gpu), 1e-6, residual=r.to(gpu))
    want, want_res = M.rms_norm_residual(x, r, w, 1e-6)
    _close(out, want, "residual out")
    assert torch.equal(res.cpu().view(torch.int16), want_res.view(torch.int16))  # bf16(x + r)


def test_add_rmsnorm_in_place(gpu):
    x, r = _rand((16, 1024), 1).to(gpu), _rand((16, 1024), 2).to(gpu)
    w = torch.ones(1024, dtype=torch.bfloat16, device=gpu)
    want, want_res = M.rms_norm_residual(x.cpu(), r.cpu(), w.cpu(), 1e-6)
    out, res = pagedkv.add_rmsnorm(x, w, 1e-6, residual=r, out=x)
    assert out.data_ptr() == x.data_ptr()
    _close(out, want, "in place")
    assert torch.equal(res.cpu().view(torch.int16), want_res.view(torch.int16))


@pytest.mark.parametrize("rows,inter", [(50, 3072), (1, 8), (257, 1024)])
def test_silu_and_mul_matches_oracle(gpu, rows, inter):
    x = _rand((rows, 2 * inter), rows, 3.0)
    got = pagedkv.silu_and_mul(x.to(gpu))
    _close(got, M.silu_and_mul(x), "silu")


def _greedy_check(got, hidden, w, cu=None):
    x = hidden.float()
    if cu is not None:
        x = x[cu[1:].long() - 1]
    logits = (x.double() @ w.double().T).to(torch.bfloat16)
    want = M.first_argmax(logits.float())
    got = got.cpu().long()
    rows = torch.arange(len(got))
    d = ulp_diff(logits[rows, got], logits[rows, want])
    assert int(d.max()) <= 1, f"chosen logit {int(d.max())} ulp below the max"
    assert float((got == want).float().mean()) >= 0.97


@pytest.mark.parametrize("rows,vocab", [(5, VOCAB), (40, VOCAB), (100, VOCAB), (300, 20011)])
def test_lm_head_greedy_matches_oracle(gpu, rows, vocab):
    w = _rand((vocab, HIDDEN), 11, 0.02)
    h = _rand((rows, HIDDEN), rows)
    got = pagedkv.lm_head_greedy(h.to(gpu), w.to(gpu))
    _greedy_check(got, h, w)


def test_lm_head_greedy_selects_last_rows_and_skips_padding(gpu):
    w = _rand((VOCAB, HIDDEN), 12, 0.02)
    h = _rand((9, HIDDEN), 13)
    cu = torch.tensor([0, 4, 5, 9], dtype=torch.int32)
    got = pagedkv.lm_head_greedy(h.to(gpu), w.to(gpu), cu.to(gpu))
    _greedy_check(got, h, w, cu)
    # zeroed tail (graph padding): sequences without rows get all-zero logits -> id 0
    cu_pad = torch.tensor([0, 4, 9, 0, 0], dtype=torch.int32)
    got = pagedkv.lm_head_greedy(h.to(gpu), w.to(gpu), cu_pad.to(gpu))
    _greedy_check(got[:2], h, w, cu_pad[:3])
    assert got[2:].tolist() == [0, 0]


def test_lm_head_greedy_one_hot_ties(gpu):
    w = torch.zeros(1000, HIDDEN)
    for v in range(1000):
        w[v, v % 8] = 1.0
    h = torch.zeros(3, HIDDEN)
    h[0, 5] = 2.0
    h[1, :8] = torch.tensor([1.0, 3.0, 3.0, 0.0, -1.0, 2.0, 0.5, 3.0])
    h[2, :8] = -1.0
    got = pagedkv.lm_head_greedy(h.to(torch.bfloat16).to(gpu), w.to(torch.bfloat16).to(gpu))
    assert got.tolist() == [5, 1, 0]
