"""GPU parity of the decode-step linear layers (pk_linear, pk_linear_add_rmsnorm) through
the C-ABI, on the projections of Qwen3-0.6B and on edge shapes.

References:
  * the linear output: the fp64 dot products rounded once to bf16 (what F.linear's bf16
    result approximates). The kernel accumulates in fp32 in its own order, so every
    element must lie within 1 bf16 ulp of the fp64 value plus the worst-case fp32
    summation error k * 2^-24 * sum_k |x w| (large, in ulps, only where the sum cancels
    to near zero), and >= 99.5% of elements must be bit-identical to the rounded fp64
    value. A transposed operand, a wrong row or k index, or a dropped split breaks both
    by orders of magnitude.
  * SiLU * mul and residual RMSNorm epilogues: the oracle's ops (oracle/model_ops.py)
    applied to the library's own linear output (checked above against fp64); bar <= 1 ulp
    and identical on >= 99% (as for the standalone norm / activation kernels).
  * composition: the fused entry points equal the library's own unfused sequence bit for
    bit (same split of K, same sums, same rounding points).
"""
import pytest
import torch

import pagedkv
from oracle import model_ops as M
from test_oracle_producer import ulp_diff

pytestmark = pytest.mark.gpu

# Qwen3-0.6B projections: (n_out, k); gate/up is (inter, k) per half
QKV, O, GATE_UP, DOWN = (4096, 1024), (1024, 2048), (3072, 1024), (1024, 3072)
ROWS = [1, 7, 32, 33, 64, 100, 128]


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _ref_linear(x, w):
    return (x.double() @ w.double().T).to(torch.bfloat16)


def _close_linear(got, x, w, what, frac=0.995):
    """got vs the fp64 product: |got - ref| <= ulp(ref) + k 2^-24 sum|x w| everywhere, and
    bit-identical to bf16(ref) on >= frac of the elements."""
    got = got.cpu().double()
    exact = x.double() @ w.double().T
    mag = x.double().abs() @ w.double().abs().T
    ref = exact.to(torch.bfloat16)
    ulp = (ref.double().abs() * 2.0 ** -7).clamp_min(2.0 ** -133)
    bound = ulp + x.shape[1] * 2.0 ** -24 * mag
    excess = ((got - exact).abs() - bound).max().item()
    assert excess <= 0, f"{what}: error exceeds the fp32 summation bound by {excess:.3e}"
    same = float((got == ref.double()).double().mean())
    assert same >= frac, f"{what}: only {same:.4f} identical to the rounded fp64 product"


def _close(got, want, what, frac=0.99):
    d = ulp_diff(got.cpu(), want.cpu())
    assert int(d.max()) <= 1, f"{what}: max ulp {int(d.max())}"
    same = float((d == 0).float().mean())
    assert same >= frac, f"{what}: only {same:.4f} identical"


def _bits(a, b):
    return torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("shape", [QKV, O, DOWN, (96, 256), (160, 512)])
def test_linear_matches_fp64(gpu, rows, shape):
    n_out, k = shape
    x, w = _rand((rows, k), rows), _rand((n_out, k), n_out + k, 0.02)
    print(f"[linear] rows={rows} n_out={n_out} k={k}", flush=True)
    got = pagedkv.linear(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    _close_linear(got, x, w, f"linear {rows}x{shape}")


@pytest.mark.parametrize("rows", [1, 33, 128])
def test_linear_silu_mul_matches_oracle(gpu, rows):
    inter, k = GATE_UP
    x, w = _rand((rows, k), rows), _rand((2 * inter, k), 9, 0.05)
    print(f"[linear_silu_mul] rows={rows}", flush=True)
    xg, wg = x.to(gpu), w.to(gpu)
    got = pagedkv.linear_silu_mul(xg, wg)
    gate, up = pagedkv.linear(xg, wg[:inter]), pagedkv.linear(xg, wg[inter:])
    unfused = pagedkv.silu_and_mul(torch.cat([gate, up], dim=1))
    torch.cuda.synchronize()
    _close_linear(gate, x, w[:inter], f"gate rows={rows}")
    _close_linear(up, x, w[inter:], f"up rows={rows}")
    want = M.silu_and_mul(torch.cat([gate, up], dim=1).cpu())
    _close(got, want, f"silu_mul rows={rows}")
    # bit-identical to the unfused library sequence (the halves use the same K split)
    assert _bits(got, unfused)


@pytest.mark.parametrize("rows", [1, 31, 64, 128])
@pytest.mark.parametrize("shape", [O, DOWN, (1024, 256)])
def test_linear_add_rmsnorm_matches_oracle(gpu, rows, shape):
    hidden, k = shape
    x, w = _rand((rows, k), rows + 3), _rand((hidden, k), 5, 0.03)
    res = _rand((rows, hidden), rows + 4, 2.0)
    nw = (_rand((hidden,), 6, 0.3).float() + 1).to(torch.bfloat16)
    print(f"[linear_add_rmsnorm] rows={rows} shape={shape}", flush=True)
    xg, wg, rg, nwg = x.to(gpu), w.to(gpu), res.to(gpu), nw.to(gpu)
    out, res_out = pagedkv.linear_add_rmsnorm(xg, wg, rg, nwg, 1e-6)
    h = pagedkv.linear(xg, wg)
    u_out, u_res = pagedkv.add_rmsnorm(h, nwg, 1e-6, residual=rg)
    torch.cuda.synchronize()
    _close_linear(h, x, w, f"linear rows={rows} shape={shape}")
    want, want_res = M.rms_norm_residual(h.cpu(), res, nw, 1e-6)
    _close(out, want, "normed")
    _close(res_out, want_res, "residual")
    # bit-identical to linear followed by the standalone residual RMSNorm kernel
    assert _bits(out, u_out) and _bits(res_out, u_res)


def test_add_rmsnorm_residual_in_place(gpu):
    hidden, k = DOWN
    x, w = _rand((48, k), 1).to(gpu), _rand((hidden, k), 2, 0.02).to(gpu)
    res = _rand((48, hidden), 3).to(gpu)
    nw = torch.ones(hidden, dtype=torch.bfloat16, device=gpu)
    want, want_res = pagedkv.linear_add_rmsnorm(x, w, res, nw, 1e-6)
    out, res_out = pagedkv.linear_add_rmsnorm(x, w, res, nw, 1e-6, residual_out=res)
    torch.cuda.synchronize()
    assert res_out.data_ptr() == res.data_ptr()
    assert _bits(out, want) and _bits(res_out, want_res)


def test_strided_rows(gpu):
    """x and out are column slices of wider row-major buffers (row stride > row length)."""
    n_out, k = QKV
    big_x = _rand((40, k + 512), 11).to(gpu)
    w = _rand((n_out, k), 12, 0.02).to(gpu)
    out = torch.zeros(40, n_out + 64, dtype=torch.bfloat16, device=gpu)
    x = big_x[:, 256:256 + k]
    pagedkv.linear(x, w, out=out[:, :n_out])
    torch.cuda.synchronize()
    _close_linear(out[:, :n_out], x.cpu(), w.cpu(), "strided")
    assert torch.count_nonzero(out[:, n_out:]) == 0  # columns past n_out untouched


def test_deterministic_and_shared_workspace(gpu):
    """Repeated calls are bit-identical, also when a call of another shape uses the same
    scratch in between."""
    x = _rand((128, 1024), 21).to(gpu)
    w = _rand((2 * 3072, 1024), 22, 0.02).to(gpu)
    x2, w2 = _rand((77, 3072), 23).to(gpu), _rand((1024, 3072), 24, 0.02).to(gpu)
    nbytes = max(pagedkv.linear_workspace_bytes(128, 3072, 1024, 1), pagedkv.linear_workspace_bytes(77, 1024, 3072))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=gpu)
    a = pagedkv.linear_silu_mul(x, w, workspace=ws)
    pagedkv.linear(x2, w2, workspace=ws)
    b = pagedkv.linear_silu_mul(x, w, workspace=ws)
    c = pagedkv.linear_silu_mul(x, w)
    torch.cuda.synchronize()
    assert _bits(a, b) and _bits(a, c)


def test_rejects_large_batches(gpu):
    with pytest.raises(ValueError):
        pagedkv.linear(torch.zeros(129, 256, dtype=torch.bfloat16, device=gpu),
                       torch.zeros(32, 256, dtype=torch.bfloat16, device=gpu))
