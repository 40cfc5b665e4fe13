"""Pins the CPU oracle (oracle/paged_kv.py) before anything is compared against it.

The reference ships no tests or golden vectors (its attention arithmetic lives in
the absent flash-attn binary), so the oracle is pinned by:
  * fp64 brute force on the known-answer cases (tests/golden);
  * closed forms: Lq = Lk = 1 gives V[0]; K = 0 gives the running mean of the visible
    V rows; constant V rows give the constant; a two-key softmax with known scores;
    per-kv-head constant V identifies the GQA map; the store/gather closed forms;
  * invariants: physical-block relabelling, shared vs duplicated prefix blocks,
    decode == last prefill row, flat == paged;
  * planted mistakes: each plausible error in the oracle (top-left causal alignment,
    GQA h % Hkv, dropped scale, storing -1 slots) must make one of the checks fail.
"""
import numpy as np
import pytest
import torch

import oracle
import oracle.paged_kv as opk
from golden.cases import CASES, BS, D, bf16_bits_to_f64, build_case, input_digest

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def _i32(a):
    return torch.from_numpy(np.asarray(a, dtype=np.int32).copy())


def oracle_on_case(case):
    bt = _i32(case["block_table"]) if case["paged"] else None
    return oracle.varlen_attention(_bf16(case["q"]), _bf16(case["k"]), _bf16(case["v"]),
                                   _i32(case["cu_q"]), _i32(case["cu_k"]), case["scale"],
                                   case["causal"], bt).numpy()


# ---------------------------------------------------------------- checks -----
# Each check raises AssertionError on a mismatch; the planted-mistake tests call them
# with a broken oracle and require that failure.

def check_kat(name):
    case = build_case(name)
    ref = np.load(GOLDEN / f"kat_{name}.npz")
    assert str(ref["digest"]) == input_digest(case), "input generator changed: rerun make_golden.py"
    got = oracle_on_case(case)
    np.testing.assert_allclose(got, ref["out"], atol=2e-5, rtol=0)


def _single(lq, lk, hq=4, hkv=2, d=16, seed=0, k=None, v=None, scale=None, causal=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(lq, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(lk, hkv, d, generator=g).to(torch.bfloat16) if k is None else k
    v = torch.randn(lk, hkv, d, generator=g).to(torch.bfloat16) if v is None else v
    cu_q = torch.tensor([0, lq], dtype=torch.int32)
    cu_k = torch.tensor([0, lk], dtype=torch.int32)
    return q, k, v, oracle.varlen_attention(q, k, v, cu_q, cu_k, scale, causal)


def check_single_key():
    q, k, v, out = _single(1, 1)
    heads = torch.tensor([0, 0, 1, 1])
    assert torch.equal(out, v[0].float()[heads].unsqueeze(0))


def check_zero_keys_running_mean():
    # K = 0: all scores equal, so row i is the mean of the V rows it sees; with
    # Lq = 5, Lk = 12 row i sees keys 0 .. i + 7 under bottom-right alignment.
    lq, lk, hkv, d = 5, 12, 2, 16
    k = torch.zeros(lk, hkv, d, dtype=torch.bfloat16)
    q, _, v, out = _single(lq, lk, k=k)
    vv = v.double().numpy()
    for i in range(lq):
        want = vv[: i + (lk - lq) + 1].mean(axis=0)           # (hkv, d)
        np.testing.assert_allclose(out[i].numpy(), want[[0, 0, 1, 1]], atol=1e-5)


def check_constant_values():
    lk = 9
    v = torch.full((lk, 2, 16), 0.375, dtype=torch.bfloat16)
    _, _, _, out = _single(3, lk, v=v)
    assert torch.allclose(out, torch.full_like(out, 0.375), atol=1e-6)


def check_two_key_softmax_scale():
    # q . k0 = 0, q . k1 = 8 per head, default scale 1/sqrt(16): p1 = sigmoid(8 / 4)
    d = 16
    q = torch.zeros(1, 2, d, dtype=torch.bfloat16)
    q[0, :, 0] = 2.0
    k = torch.zeros(2, 1, d, dtype=torch.bfloat16)
    k[1, 0, 0] = 4.0
    v = torch.zeros(2, 1, d, dtype=torch.bfloat16)
    v[1, 0, :] = 1.0
    cu = torch.tensor([0, 1], dtype=torch.int32)
    cuk = torch.tensor([0, 2], dtype=torch.int32)
    out = oracle.varlen_attention(q, k, v, cu, cuk, None, True)
    p1 = 1.0 / (1.0 + np.exp(-8.0 / 4.0))
    np.testing.assert_allclose(out[0, :, 0].numpy(), [p1, p1], rtol=1e-6)


def check_gqa_map():
    # V of kv head g is the constant g: output head h must equal h // (Hq / Hkv)
    hq, hkv, lk = 8, 4, 6
    v = torch.arange(hkv, dtype=torch.float32).view(1, hkv, 1).expand(lk, hkv, 16).to(torch.bfloat16)
    _, _, _, out = _single(2, lk, hq=hq, hkv=hkv, v=v)
    want = (torch.arange(hq) // (hq // hkv)).float()
    assert torch.allclose(out[:, :, 0], want.expand(2, hq))


def check_store_closed_form():
    nb, bs, hkv, d, n = 4, 8, 2, 8, 10
    g = torch.Generator().manual_seed(3)
    key = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
    value = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
    sentinel = torch.full((nb, bs, hkv, d), -7.0, dtype=torch.bfloat16)
    kc, vc = sentinel.clone(), sentinel.clone()
    slots = torch.tensor([5, -1, 31, 0, -1, 12, 13, 30, -1, 7], dtype=torch.int32)
    oracle.store_kvcache(key, value, kc, vc, slots)
    rows_k, rows_v = kc.view(-1, hkv, d), vc.view(-1, hkv, d)
    written = set()
    for i, s in enumerate(slots.tolist()):
        if s == -1:
            continue
        written.add(s)
        assert torch.equal(rows_k[s], key[i]) and torch.equal(rows_v[s], value[i])
    for s in range(nb * bs):
        if s not in written:
            assert torch.equal(rows_k[s], sentinel.view(-1, hkv, d)[s])
            assert torch.equal(rows_v[s], sentinel.view(-1, hkv, d)[s])


# ------------------------------------------------------------ the tests -----

@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_bruteforce_kat(name):
    check_kat(name)


@pytest.mark.parametrize("check", [check_single_key, check_zero_keys_running_mean,
                                   check_constant_values, check_two_key_softmax_scale,
                                   check_gqa_map, check_store_closed_form])
def test_closed_forms(check):
    check()


def test_store_strided_value_rows():
    # v as a view into a fused qkv row (row stride 4 * row) is stored bit-exactly
    n, hkv, d = 6, 2, 8
    qkv = torch.randn(n, 4 * hkv * d).to(torch.bfloat16)
    v = qkv[:, 3 * hkv * d:].view(n, hkv, d)
    k = qkv[:, 2 * hkv * d:3 * hkv * d].reshape(n, hkv, d).clone()
    kc = torch.zeros(2, 4, hkv, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([7, 6, 5, 4, 3, 2], dtype=torch.int32)
    oracle.store_kvcache(k, v, kc, vc, slots)
    assert torch.equal(vc.view(-1, hkv, d)[slots.long()], v)


def test_gather_closed_form():
    case = build_case("mixed4")
    cache = _bf16(case["k"])
    bt = _i32(case["block_table"])
    cu = _i32(case["cu_k"])
    flat = oracle.gather_kv(cache, bt, cu)
    rows = cache.view(-1, case["hkv"], D)
    for b, lk in enumerate(case["k_lens"]):
        for t in (0, lk // 2, lk - 1):
            s = int(bt[b, t // BS]) * BS + t % BS
            assert torch.equal(flat[int(cu[b]) + t], rows[s])


def test_block_relabelling_is_bit_invariant():
    case = build_case("prefill2")
    base = oracle_on_case(case)
    nb = case["k"].shape[0]
    perm = np.random.default_rng(5).permutation(nb)       # new position of old block j
    k2 = np.empty_like(case["k"])
    v2 = np.empty_like(case["v"])
    k2[perm] = case["k"]
    v2[perm] = case["v"]
    bt2 = np.where(case["block_table"] >= 0, perm[np.maximum(case["block_table"], 0)], -1)
    relabelled = dict(case, k=k2, v=v2, block_table=bt2.astype(np.int32))
    assert np.array_equal(oracle_on_case(relabelled), base)


def test_shared_prefix_equals_duplicated_prefix():
    # two sequences reading the same physical prefix blocks == reading private copies
    case = build_case("decode3")
    bt = case["block_table"].copy()
    shared = bt[2, :2].copy()            # sequence 2's first two blocks (128 keys)
    bt[1, :2] = shared                   # sequence 1 (70 keys) now shares them
    a = dict(case, block_table=bt)
    k2 = np.concatenate([case["k"], case["k"][shared]])
    v2 = np.concatenate([case["v"], case["v"][shared]])
    nb = case["k"].shape[0]
    bt_dup = bt.copy()
    bt_dup[1, :2] = [nb, nb + 1]          # private copies of the same bits
    b = dict(case, k=k2, v=v2, block_table=bt_dup)
    assert np.array_equal(oracle_on_case(a), oracle_on_case(b))


def test_decode_equals_last_prefill_row():
    case = build_case("prefill2")
    full = oracle_on_case(case)
    # the same keys, queried only by the last row of sequence 1 (Lq = 1)
    lq1 = case["q_lens"][1]
    last = case["q"][case["cu_q"][2] - 1: case["cu_q"][2]]
    dec = dict(case, q=last, cu_q=np.array([0, 0, 1], np.int32))
    got = oracle_on_case(dec)
    np.testing.assert_allclose(got[0], full[case["cu_q"][1] + lq1 - 1], atol=1e-6)


def test_flat_equals_paged():
    case = build_case("prefill2")
    paged = oracle_on_case(case)
    k_flat = oracle.gather_kv(_bf16(case["k"]), _i32(case["block_table"]), _i32(case["cu_k"]))
    v_flat = oracle.gather_kv(_bf16(case["v"]), _i32(case["block_table"]), _i32(case["cu_k"]))
    flat = oracle.varlen_attention(_bf16(case["q"]), k_flat, v_flat, _i32(case["cu_q"]),
                                   _i32(case["cu_k"]), case["scale"], True, None).numpy()
    assert np.array_equal(flat, paged)


def test_padded_sequences_are_skipped():
    case = build_case("padded")
    out = oracle_on_case(case)
    assert out.shape[0] == sum(case["q_lens"])
    ref = np.load(GOLDEN / "kat_padded.npz")["out"]
    np.testing.assert_allclose(out, ref, atol=2e-5)


def test_bf16_helpers_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38], dtype=np.float32)
    from golden.cases import f32_to_bf16_bits
    got = bf16_bits_to_f64(f32_to_bf16_bits(x))
    want = torch.from_numpy(x).to(torch.bfloat16).double().numpy()
    assert np.array_equal(got, want)


# ------------------------------------------------------ planted mistakes -----

def _top_left_visible(lq, lk, causal):
    i = torch.arange(lq).unsqueeze(1)
    t = torch.arange(lk).unsqueeze(0)
    return torch.ones(lq, lk, dtype=torch.bool) if not causal else t <= i


def _modulo_heads(num_heads, num_kv_heads):
    return torch.arange(num_heads) % num_kv_heads


@pytest.mark.parametrize("attr,bad,checks", [
    ("visible", _top_left_visible, [check_zero_keys_running_mean, lambda: check_kat("prefill2")]),
    ("kv_head_of", _modulo_heads, [check_gqa_map, lambda: check_kat("gqa4")]),
    ("default_scale", lambda d, s: 1.0, [check_two_key_softmax_scale]),
    ("_keep_slots", lambda s: np.ones_like(s, dtype=bool), [check_store_closed_form]),
])
def test_planted_mistakes_are_caught(monkeypatch, attr, bad, checks):
    monkeypatch.setattr(opk, attr, bad)
    for chk in checks:
        with pytest.raises(AssertionError):
            chk()
