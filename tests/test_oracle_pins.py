"""Pins of the CPU oracle (oracle/) -- no GPU.

Each check is independent of the oracle's own code path: the reference
repository's test formulas (tests/test_moe_w8a8.py:40-69,
tests/test_i8gemm.py:18-37, tests/test_deepseek_v4_w8a8.py:19-50,
tests/test_moe_w8a8.py:238-242) evaluated with torch, known answers (ties),
exact integer arithmetic, closed forms (2^(i/64)), libm exp, and brute force
on small inputs.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from tests import helpers as H


# ------------------------------------------------------------------ bf16 --

def test_bf16_rounding_matches_torch(oracle_lib):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([1.00390625, 1.01171875, -1.00390625, 0.0, -0.0], np.float32)])  # exact ties
    mine = oracle_lib.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(mine, ref)
    assert oracle_lib.lib().orc_f32_to_bf16(1.00390625) == 0x3F80  # tie to even (down)
    assert oracle_lib.lib().orc_f32_to_bf16(1.01171875) == 0x3F82  # tie to even (up)


# ----------------------------------------------------------------- FEXPA --

def test_fexpa_table_is_nearest_2_pow_i_over_64(oracle_lib):
    table = oracle_lib.fexpa_table()
    for i in range(64):
        # 2^(i/64) * 2^23 to 30 digits with exact rounding of the closed form
        v = Fraction(int(round(2 ** (i / 64) * 2**53)), 2**30)
        expect = int(v + Fraction(1, 2)) - 2**23
        assert table[i] == expect, i
    assert table[1] == 0x0164D2 and table[32] == 0x3504F3  # sqrt(2) fraction


def test_fexpa_exp_matches_libm(oracle_lib):
    g = np.concatenate([np.linspace(-80, 80, 4001), np.array([0.0, 1e-7, -1e-7, 10.0, -10.0])])
    for v in g:
        got = oracle_lib.fexpa_exp_neg(float(np.float32(v)))
        ref = math.exp(-float(np.float32(v)))
        assert abs(got - ref) <= 3e-6 * ref, (v, got, ref)
    # clamp to +-87 (kernels.cpp:201)
    assert oracle_lib.fexpa_exp_neg(200.0) == oracle_lib.fexpa_exp_neg(87.0)
    assert oracle_lib.fexpa_exp_neg(-200.0) == oracle_lib.fexpa_exp_neg(-87.0)


# ------------------------------------------------------- row quantisation --

def test_quant_half_away_known_answers(oracle_lib):
    x = np.zeros((2, 16), np.float32)
    x[0, :6] = [127.0, 0.5, 1.5, -0.5, 2.5, -2.5]  # scale exactly 1: ties
    q, s = oracle_lib.quant_rows_away(H.bf16_bits(x))
    assert s[0] == 1.0 and s[1] == 1.0  # zero row: scale 1
    assert list(q[0, :6]) == [127, 1, 2, -1, 3, -3]  # rinta: half away from zero
    assert (q[1] == 0).all()


def test_quant_half_away_closed_form(oracle_lib):
    rng = np.random.default_rng(1)
    x = H.bf16_bits(rng.standard_normal((64, 300)).astype(np.float32) * 4)
    q, s = oracle_lib.quant_rows_away(x)
    xf = H.bits_to_f32(x)
    m = np.abs(xf).max(axis=1)
    scale = np.where(m > 0, (m / np.float32(127)).astype(np.float32), np.float32(1))
    inv = (np.float32(1) / scale).astype(np.float32)
    v = np.clip((xf * inv[:, None]).astype(np.float32), -127, 127).astype(np.float64)
    expect = np.trunc(v + np.copysign(0.5, v)).astype(np.int8)
    np.testing.assert_array_equal(s, scale)
    np.testing.assert_array_equal(q, expect)


def test_quant_ties_to_even_matches_reference_tests(oracle_lib):
    # tests/test_deepseek_v4_w8a8.py:40-50 known answer
    x = np.zeros((2, 16), np.float32)
    x[0, :5] = [127.0, 0.5, 1.5, -0.5, -1.5]
    q, _ = oracle_lib.quant_rows_even(H.bf16_bits(x))
    assert list(q[0, :5]) == [127, 0, 2, 0, -2]
    # tests/test_i8gemm.py:25-28 closed form, bf16 and fp32 rows
    rng = np.random.default_rng(2)
    for xin in (H.bf16_bits(rng.standard_normal((9, 31)).astype(np.float32)),
                rng.standard_normal((9, 31)).astype(np.float32)):
        q, s = oracle_lib.quant_rows_even(xin)
        t = torch.from_numpy(H.bits_to_f32(xin) if xin.dtype == np.uint16 else xin)
        mx = t.abs().amax(dim=-1)
        ts = torch.where(mx > 0, mx / 127.0, torch.ones_like(mx))
        tq = torch.round(t / ts.unsqueeze(-1)).clamp(-128, 127).to(torch.int8)
        np.testing.assert_array_equal(q, tq.numpy())
        np.testing.assert_array_equal(s, ts.numpy())


def test_weight_quant_matches_reference_test(oracle_lib):
    # tests/test_moe_w8a8.py:233-251 closed form
    g = torch.Generator().manual_seed(29)
    w = (torch.randn((2, 32, 16), generator=g) * 0.1).to(torch.bfloat16)
    w[0, 3] = 0  # zero channel -> scale 1
    fp32 = w.float()
    mx = fp32.abs().amax(dim=-1, keepdim=True)
    sc = torch.where(mx > 0, mx / 127.0, torch.ones_like(mx))
    tq = (fp32 / sc).round().clamp(-127, 127).to(torch.int8)
    q, s = oracle_lib.quant_weight_rows(w.view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(q, tq.numpy())
    np.testing.assert_array_equal(s, sc.squeeze(-1).numpy())


# -------------------------------------------------------------- routing --

@pytest.mark.parametrize("tokens,experts,k,renorm,scale", [(5, 8, 2, True, 1.0), (64, 256, 8, True, 2.5),
                                                            (33, 384, 8, False, 1.0), (7, 1024, 64, True, 1.0)])
def test_router_oracle_matches_torch_float64_and_brute_force(oracle_lib, tokens, experts, k, renorm, scale):
    rng = np.random.default_rng(experts + k)
    x = rng.standard_normal((tokens, experts)).astype(np.float32)
    ids, w = oracle_lib.router_topk(x, k, renormalize=renorm, scale=scale)
    # torch float64: softmax -> topk (sorted) -> renormalise -> scale
    p = torch.softmax(torch.from_numpy(x).double(), dim=1)
    tw, ti = torch.topk(p, k, dim=1, sorted=True)
    if renorm:
        tw = tw / tw.sum(dim=1, keepdim=True)
    np.testing.assert_array_equal(ids, ti.numpy())
    np.testing.assert_allclose(w, (tw * scale).numpy(), rtol=2e-6, atol=1e-9)
    # brute force selection order on the first rows
    for t in range(min(tokens, 3)):
        expect = sorted(range(experts), key=lambda e: (-float(x[t, e]), e))[:k]
        assert list(ids[t]) == expect


def test_router_oracle_ties_take_lower_id(oracle_lib):
    x = np.array([[1.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    ids, w = oracle_lib.router_topk(x, 2, scale=2.0)
    assert ids.tolist() == [[1, 2], [0, 1]]
    np.testing.assert_allclose(w, [[1.0, 1.0], [1.0, 1.0]], rtol=1e-7)


@pytest.mark.parametrize("tokens,top_k,experts,shared", [(1, 1, 1, -1), (37, 2, 4, -1), (50, 8, 17, 16),
                                                          (300, 6, 9, 8)])
def test_route_build_matches_stable_argsort_and_brute_force(oracle_lib, tokens, top_k, experts, shared):
    rng = np.random.default_rng(tokens)
    routed = experts - 1 if shared >= 0 else experts
    ids = rng.integers(0, routed, size=(tokens, top_k)).astype(np.int64)
    counts, offsets, sorted_routes, bad = oracle_lib.route_build(ids, experts, shared)
    kt = top_k + (1 if shared >= 0 else 0)
    flat = np.concatenate([ids, np.full((tokens, 1), shared)], axis=1).reshape(-1) if shared >= 0 else ids.reshape(-1)
    # brute force: per expert, ascending route index
    expect = [r for e in range(experts) for r in range(tokens * kt) if flat[r] == e]
    np.testing.assert_array_equal(sorted_routes, expect)
    # torch stable argsort gives the same permutation
    np.testing.assert_array_equal(sorted_routes, torch.argsort(torch.from_numpy(flat), stable=True).numpy())
    np.testing.assert_array_equal(counts, np.bincount(flat, minlength=experts))
    assert bad == 0 and offsets[-1] == tokens * kt


def test_route_build_counts_invalid_ids(oracle_lib):
    ids = np.array([[0, 5], [-1, 1]], np.int64)
    counts, offsets, sorted_routes, bad = oracle_lib.route_build(ids, 4)
    assert bad == 2 and list(sorted_routes) == [0, 3] and offsets[-1] == 2


# ---------------------------------------------------------------- W8A8 --

def _reference_moe_w8a8(input, q13, s13, q2, s2, topk_weights, topk_ids):
    """tests/test_moe_w8a8.py:40-69 (per token, torch.exp, division, round half even)."""
    def quantize_row(row):
        row = row.float()
        scale = max(float(row.abs().max()) / 127.0, 1.0e-30)
        return (row / scale).round().clamp(-127, 127).to(torch.int32), scale

    tokens, hidden = input.shape
    inter = q2.size(2)
    output = torch.zeros((tokens, hidden), dtype=torch.float32)
    for token in range(tokens):
        input_q, input_scale = quantize_row(input[token])
        for slot in range(topk_ids.size(1)):
            expert = int(topk_ids[token, slot])
            w13 = (input_q @ q13[expert].to(torch.int32).T).float() * input_scale * s13[expert]
            gate = w13[:inter].clamp(max=10.0)
            up = w13[inter:].clamp(-10.0, 10.0)
            activated = (gate * up / (1.0 + torch.exp(-gate))).to(torch.bfloat16)
            intermediate_q, intermediate_scale = quantize_row(activated)
            route = (intermediate_q @ q2[expert].to(torch.int32).T).float() * intermediate_scale * s2[expert]
            output[token].add_(route, alpha=float(topk_weights[token, slot]))
    return output.to(torch.bfloat16)


@pytest.mark.parametrize("experts", [1, 2])
def test_w8a8_oracle_matches_reference_test(oracle_lib, experts):
    """The exact inputs and tolerance of test_w8a8_plan_v2_matches_dynamic_quantization_reference."""
    generator = torch.Generator().manual_seed(23)
    hidden, intermediate, tokens = 64, 64, 48
    q13 = torch.randint(-12, 13, (experts, 2 * intermediate, hidden), dtype=torch.int8, generator=generator)
    q2 = torch.randint(-12, 13, (experts, hidden, intermediate), dtype=torch.int8, generator=generator)
    s13 = torch.rand((experts, 2 * intermediate), generator=generator) * 0.003 + 0.0005
    s2 = torch.rand((experts, hidden), generator=generator) * 0.003 + 0.0005
    inp = (torch.randn((tokens, hidden), generator=generator) * 0.3).to(torch.bfloat16)
    ids = torch.tensor([[t % experts] for t in range(tokens)], dtype=torch.int64)
    w = torch.ones((tokens, 1), dtype=torch.float32)
    got = oracle_lib.w8a8_forward(inp.view(torch.int16).numpy().view(np.uint16), ids.numpy(), w.numpy(),
                                  q13.numpy(), s13.numpy(), q2.numpy(), s2.numpy())
    expect = _reference_moe_w8a8(inp, q13, s13, q2, s2, w, ids)
    got_t = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16)
    torch.testing.assert_close(got_t.float(), expect.float(), rtol=0.0, atol=3.0e-6)


def test_w8a8_oracle_multislot_shared_close_to_reference_formula(oracle_lib):
    """top-3 plus a shared expert (weight 1, routed x2.5) against the same per-token formula."""
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(41, 20, 128, 64, 6, 3, int_range=12)
    ids = np.minimum(ids, 4)
    got = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=5, routed_scale=2.5)
    ids_c = np.concatenate([ids, np.full((20, 1), 5)], 1)
    w_c = np.concatenate([w * np.float32(2.5), np.ones((20, 1), np.float32)], 1)
    expect = _reference_moe_w8a8(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16), torch.from_numpy(q13),
                                 torch.from_numpy(s13), torch.from_numpy(q2), torch.from_numpy(s2),
                                 torch.from_numpy(w_c), torch.from_numpy(ids_c))
    g = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float()
    # the reference formula differs in exp, tie rounding and division; allow
    # one bf16 ulp of the output scale
    torch.testing.assert_close(g, expect.float(), rtol=1e-2, atol=2e-2 * float(expect.float().abs().max()))


def test_w8a8_oracle_stage_accumulators_are_exact_integer_gemms(oracle_lib):
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(17, 12, 192, 96, 4, 2)
    out, d = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, dumps=True)
    xq, xs = oracle_lib.quant_rows_away(x)
    for t in range(12):
        for s in range(2):
            r = t * 2 + s
            e = ids[t, s]
            np.testing.assert_array_equal(d["acc13"][r], xq[t].astype(np.int64) @ q13[e].astype(np.int64).T)
            np.testing.assert_array_equal(d["acc2"][r], d["q2"][r].astype(np.int64) @ q2[e].astype(np.int64).T)
    # requant of the bf16 intermediate is the activation quantiser
    q2r, s2r = oracle_lib.quant_rows_away(d["y"])
    np.testing.assert_array_equal(q2r, d["q2"])
    np.testing.assert_array_equal(s2r, d["s2row"])
    # merge: ordered fma over slots
    ro = d["route_out"]
    for t in range(12):
        acc32 = np.zeros(192, np.float32)
        for s in range(2):  # fma: exact product in float64, one rounding to float32
            acc32 = (ro[t * 2 + s].astype(np.float64) * np.float64(w[t, s]) + acc32.astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(out[t], oracle_lib.f32_to_bf16_bits(acc32))


# --------------------------------------------------------------- i8gemm --

def _reference_i8gemm(x, weight_int8, weight_scale, bias=None, out_dtype=torch.float32):
    """tests/test_i8gemm.py:18-37."""
    x_2d = x.reshape(-1, x.shape[-1]).to(torch.float32)
    max_abs = x_2d.abs().amax(dim=-1)
    x_scale = torch.where(max_abs > 0, max_abs / 127.0, torch.ones_like(max_abs))
    x_q = torch.round(x_2d / x_scale.unsqueeze(-1)).clamp(-128, 127).to(torch.int8)
    acc = x_q.to(torch.int32) @ weight_int8.t().contiguous().to(torch.int32)
    scale = weight_scale.reshape(-1).to(torch.float32)
    if scale.numel() == 1:
        scale = scale.expand(weight_int8.shape[0])
    out = acc.to(torch.float32) * x_scale.unsqueeze(-1) * scale.unsqueeze(0)
    if bias is not None:
        out = out + bias.to(torch.float32)
    return out.to(out_dtype).reshape(*x.shape[:-1], weight_int8.shape[0])


@pytest.mark.parametrize("m,k,n,bf16_out", [(1, 7, 5, False), (4, 16, 8, True), (9, 31, 13, True),
                                            (24, 64, 96, False)])
def test_i8gemm_oracle_matches_reference_test(oracle_lib, m, k, n, bf16_out):
    torch.manual_seed(0)
    weight = torch.randint(-16, 17, (n, k), dtype=torch.int8)
    weight_scale = torch.rand(n, dtype=torch.float32) * 0.05 + 0.01
    bias = torch.randn(n, dtype=torch.bfloat16)
    x = torch.randn(m, k, dtype=torch.bfloat16)
    out_dtype = torch.bfloat16 if bf16_out else torch.float32
    expect = _reference_i8gemm(x, weight, weight_scale, bias=bias, out_dtype=out_dtype)
    got = oracle_lib.i8gemm(x.view(torch.int16).numpy().view(np.uint16), weight.numpy(), weight_scale.numpy(),
                            bias.float().numpy(), bf16_out)
    if bf16_out:
        np.testing.assert_array_equal(got, expect.view(torch.int16).numpy().view(np.uint16))
    else:
        np.testing.assert_array_equal(got.view(np.uint32), expect.numpy().view(np.uint32))


def test_i8gemm_oracle_scalar_scale_fp32_input():
    import oracle

    torch.manual_seed(1)
    weight = torch.randint(-8, 9, (11, 19), dtype=torch.int8)
    x = torch.randn(6, 19, dtype=torch.float32)
    expect = _reference_i8gemm(x, weight, torch.tensor(0.02), out_dtype=torch.bfloat16)
    got = oracle.i8gemm(x.numpy(), weight.numpy(), np.float32(0.02), None, True)
    np.testing.assert_array_equal(got, expect.view(torch.int16).numpy().view(np.uint16))


# ----------------------------------------------------------- BF16 oracle --

@pytest.mark.parametrize("mode", ["silu", "gelu", "swigluoai", "silu_clamp10"])
def test_bf16_activation_within_one_ulp_of_float64(oracle_lib, mode):
    rng = np.random.default_rng(3)
    gu = (rng.standard_normal((8, 64)) * 6).astype(np.float32)
    got = H.bits_to_f32(oracle_lib.bf16_activation(gu, mode)).astype(np.float64)
    g64 = gu.astype(np.float64)
    if mode == "swigluoai":
        gate, up = np.minimum(g64[:, ::2], 7), np.clip(g64[:, 1::2], -7, 7)
        ref = (up + 1) * gate / (1 + np.exp(-gate * 1.702))
    else:
        gate, up = g64[:, :32], g64[:, 32:]
        if mode == "silu_clamp10":
            gate, up = np.minimum(gate, 10), np.clip(up, -10, 10)
        if mode == "gelu":
            from scipy.special import erf

            ref = 0.5 * gate * (1 + erf(gate / math.sqrt(2))) * up
        else:
            ref = gate / (1 + np.exp(-gate)) * up
    # one bf16 ulp relative; the absolute floor covers fp32 cancellation in
    # 1 + erf(x) for large negative x, which the fp32 reference shares
    np.testing.assert_allclose(got, ref, rtol=2 ** -8, atol=1e-5)


def test_bf16_reference_matches_per_token_brute_force(oracle_lib):
    """Grouped numpy reference == per-token float64 loops (naive.py:161-272 semantics)."""
    rng = np.random.default_rng(4)
    T, Hd, F, E, k = 37, 13, 11, 4, 2
    x = rng.standard_normal((T, Hd)).astype(np.float32)
    w13 = rng.standard_normal((E, 2 * F, Hd)).astype(np.float32)
    w2 = rng.standard_normal((E, Hd, F)).astype(np.float32)
    b13 = (rng.standard_normal((E, 2 * F)) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal((E, Hd)) * 0.1).astype(np.float32)
    ids = np.array([[(i + j) % E for j in range(k)] for i in range(T)])
    w = rng.random((T, k)).astype(np.float32)
    got = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, w13_bias=b13, w2_bias=b2, activation="silu")
    ref = np.zeros((T, Hd))
    for t in range(T):
        for s in range(k):
            e = ids[t, s]
            gu = w13[e].astype(np.float64) @ x[t].astype(np.float64) + b13[e]
            y = gu[:F] / (1 + np.exp(-gu[:F])) * gu[F:]
            ref[t] += w[t, s] * (w2[e].astype(np.float64) @ y + b2[e])
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def _f32(x):
    return np.float32(x)


@pytest.mark.parametrize("kt", [2, 4, 6, 8])
def test_bf16_merge_tree_follows_reference_comment(oracle_lib, kt):
    """route_merge.cpp:54-55 states the tree: split each range at its largest
    power of two, so TopK=6 is ((0+1)+(2+3))+(4+5). Products are rounded
    first (weighted_leaf, :47-52). Inputs mix magnitudes so a left fold, a
    fused chain or another pairing round differently; the test shows that for
    each alternative on some element, and that the oracle follows the stated
    tree on every element."""
    rng = np.random.default_rng(kt)
    tokens, hidden = 3, 512
    mag = np.array([1e7, 1.0, -1e7, 3.0, 1e-3, 7.0, -5.0, 2.0], np.float32)[:kt]
    rows = (rng.standard_normal((tokens * kt, hidden)).astype(np.float32) * np.tile(mag, tokens)[:, None])
    w = rng.uniform(0.1, 2.0, tokens * kt).astype(np.float32)
    got = oracle_lib.bf16_route_merge(rows, w, kt)

    def tree(p, b, c):
        if c == 1:
            return p[b]
        left = 1
        while left * 2 < c:
            left *= 2
        return _f32(tree(p, b, left) + tree(p, b + left, c - left))

    prods = (rows.reshape(tokens, kt, hidden) * w.reshape(tokens, kt, 1)).astype(np.float32)
    want = np.empty((tokens, hidden), np.float32)
    fold = np.zeros((tokens, hidden), np.float32)
    chain = np.zeros((tokens, hidden), np.float32)
    for t in range(tokens):
        for h in range(hidden):
            want[t, h] = tree(prods[t, :, h], 0, kt)
        for s in range(kt):
            fold[t] = (fold[t] + prods[t, s]).astype(np.float32)
            chain[t] = (rows.reshape(tokens, kt, hidden)[t, s].astype(np.float64) * np.float64(w[t * kt + s])
                        + chain[t]).astype(np.float32)
    np.testing.assert_array_equal(got, oracle_lib.f32_to_bf16_bits(want))
    if kt > 2:  # for two leaves every order is the same sum
        assert not np.array_equal(want, fold)
        assert not np.array_equal(want, chain)


@pytest.mark.parametrize("kt", [1, 3, 5, 9])
def test_bf16_merge_ordered_chain_is_fused(oracle_lib, kt):
    """Other top-k: acc = fma(row, w, acc) in slot order (merge_dynamic_block,
    route_merge.cpp:78-86): equal to an exact-product float64 chain rounded
    to float32 each step, and (for kt > 1) not to the unfused form."""
    rng = np.random.default_rng(40 + kt)
    tokens, hidden = 4, 777
    rows = rng.standard_normal((tokens * kt, hidden)).astype(np.float32) * 100
    w = rng.uniform(0.1, 2.0, tokens * kt).astype(np.float32)
    got = oracle_lib.bf16_route_merge(rows, w, kt)
    r3 = rows.reshape(tokens, kt, hidden)
    acc = np.zeros((tokens, hidden), np.float32)
    unfused = np.zeros((tokens, hidden), np.float32)
    for s in range(kt):
        ws = w.reshape(tokens, kt)[:, s:s + 1]
        acc = (r3[:, s].astype(np.float64) * ws.astype(np.float64) + acc).astype(np.float32)
        unfused = ((r3[:, s] * ws).astype(np.float32) + unfused).astype(np.float32)
    np.testing.assert_array_equal(got, oracle_lib.f32_to_bf16_bits(acc))
    if kt > 1:
        assert not np.array_equal(acc, unfused)


@pytest.mark.parametrize("shared", [False, True])
def test_oracle_staged_layer_equals_forward(oracle_lib, shared):
    """The oracle's stage entry points (W13 epilogue + requant, store_w2,
    merge) around an exact int64 numpy GEMM give orc_w8a8_forward's output bit
    for bit, invalid ids included: they are the same code, factored out, which
    the whole-layer GPU checks at the BASELINE shapes use with a device GEMM."""
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(77, 23, 192, 96, 7, 3)
    ids = ids.copy()
    ids[3, 1] = 7   # out of range: dropped
    ids[5, 0] = -1
    sid = 6 if shared else -1
    ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=sid, routed_scale=2.5)
    g13 = lambda e, a: (a.astype(np.int64) @ q13[e].astype(np.int64).T).astype(np.int32)  # noqa: E731
    g2 = lambda e, a: (a.astype(np.int64) @ q2[e].astype(np.int64).T).astype(np.int32)  # noqa: E731
    got = H.w8a8_layer_staged(x, ids, w, 7, sid, 2.5, g13, g2, lambda e: s13[e], lambda e: s2[e])
    np.testing.assert_array_equal(got, ref)
