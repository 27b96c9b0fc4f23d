"""The W8A8 decode tail (requant + W2 + ordered merge in one launch) and, at one
token, the decode head (route + token-row quantisation + W13 in one launch)
of fcmoe_decode_tail.hip, against the launches they replace
(FCMOE_DECODE_TAIL_MAX_T=0) and the CPU oracle. The tail runs for one-token
batches by default and is forced here for up to two
(FCMOE_DECODE_TAIL_MAX_T=2); the head always takes one-token batches with it.

Reference semantics: the route order (kernels.cpp:583-592), quantize_bf16_row
of the token row and of the intermediate, w13_epilogue and store_w2
(csrc/moe/arm/i8mm_w8a8/kernels.cpp:211-257, 650-657) and the ordered top-k
merge (kernels.cpp:674-688). Everything is compared bit for bit: the output,
the invalid-id count, and the sorted_routes / y / q2 / s2row / route_out views
that the unfused path leaves.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _run(case, gpu, *, tail: bool, **kw):
    old = os.environ.get("FCMOE_DECODE_TAIL_MAX_T")
    os.environ["FCMOE_DECODE_TAIL_MAX_T"] = "2" if tail else "0"
    try:
        return H.gpu_w8a8_forward(*case, gpu, stages=True, **kw)
    finally:
        if old is None:
            del os.environ["FCMOE_DECODE_TAIL_MAX_T"]
        else:
            os.environ["FCMOE_DECODE_TAIL_MAX_T"] = old


def _valid_routes(ids, experts_valid, shared: bool):
    """Flat routes whose id is valid (the shared slot always is)."""
    T, k = ids.shape
    ok = (ids >= 0) & (ids < experts_valid)
    if shared:
        ok = np.concatenate([ok, np.ones((T, 1), bool)], 1)
    return np.nonzero(ok.reshape(-1))[0]


def _compare(a, b, ids, valid_experts, shared):
    (out_a, st_a), (out_b, st_b) = a, b
    np.testing.assert_array_equal(out_a, out_b)
    routes = _valid_routes(ids, valid_experts, shared)
    n = len(routes)
    np.testing.assert_array_equal(st_a["sorted_routes"][:n], st_b["sorted_routes"][:n])
    np.testing.assert_array_equal(st_a["y"][:n], st_b["y"][:n])
    np.testing.assert_array_equal(st_a["q2"][:n], st_b["q2"][:n])
    np.testing.assert_array_equal(st_a["s2row"][:n].view(np.uint32), st_b["s2row"][:n].view(np.uint32))
    np.testing.assert_array_equal(st_a["route_out"][routes].view(np.uint32), st_b["route_out"][routes].view(np.uint32))


# (seed, tokens, hidden, inter, experts incl. shared, top_k, shared)
CASES = [
    (1, 1, 256, 128, 8, 2, True),
    (2, 2, 512, 192, 16, 4, True),
    (3, 1, 1024, 80, 6, 3, False),   # I % 64 != 0: the zero-padded K tail
    (4, 2, 7168, 2048, 33, 8, True),  # DSv3 widths
    (5, 1, 256, 48, 20, 15, True),    # 16 slots, the most the tail takes
    (7, 1, 256, 48, 10, 2, True),     # one K chunk per slot
    (8, 1, 256, 128, 20, 15, True),   # 16 slots, two K chunks
    (6, 2, 768, 256, 12, 6, False),
]


@pytest.mark.parametrize("case_args", CASES, ids=[f"T{c[1]}-H{c[2]}-I{c[3]}-k{c[5]}" for c in CASES])
def test_decode_tail_matches_unfused_and_oracle(gpu, oracle_lib, case_args):
    seed, T, Hd, I, E, k, shared = case_args
    case = H.w8a8_case(seed, T, Hd, I, E, k)
    x, ids, w, q13, s13, q2, s2 = case
    sid = E - 1 if shared else -1
    if shared:
        ids = np.minimum(ids, E - 2)
        case = (x, ids, w, q13, s13, q2, s2)
    print(f"[decode-tail] T={T} H={Hd} I={I} E={E} k={k} shared={shared}", flush=True)
    fused = _run(case, gpu, tail=True, shared_id=sid, scale=2.5)
    plain = _run(case, gpu, tail=False, shared_id=sid, scale=2.5)
    ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=sid, routed_scale=2.5)
    np.testing.assert_array_equal(plain[0], ref, err_msg="unfused path vs oracle")
    np.testing.assert_array_equal(fused[0], ref, err_msg="decode tail vs oracle")
    _compare(fused, plain, ids, E, shared)


def test_decode_tail_with_dropped_routes(gpu):
    """Out-of-range ids drop their routes: the tail skips them as the merge does,
    including a token whose routed slots are all dropped (no shared expert)."""
    case = H.w8a8_case(11, 2, 512, 128, 10, 4)
    x, ids, w, q13, s13, q2, s2 = case
    ids = ids.copy()
    ids[0, 1] = 10   # == valid_experts: out of range
    ids[0, 3] = -1
    ids[1, :] = 99   # every slot of token 1
    case = (x, ids, w, q13, s13, q2, s2)
    print("[decode-tail] dropped routes", flush=True)
    fused = _run(case, gpu, tail=True, valid_experts=10)
    plain = _run(case, gpu, tail=False, valid_experts=10)
    _compare(fused, plain, ids, 10, False)
    assert fused[1]["invalid"] == plain[1]["invalid"] == 6
    assert not fused[0][1].any()  # the merge of nothing is 0


@pytest.mark.parametrize("shared", [True, False])
def test_decode_head_one_token_dropped_routes(gpu, shared):
    """One token (the head path) with out-of-range ids, and with every routed id
    out of range (only the shared slot left, or no slot at all)."""
    E = 10
    case = H.w8a8_case(31, 1, 512, 128, E, 4)
    x, ids, w, q13, s13, q2, s2 = case
    sid = E - 1 if shared else -1
    for bad in ([1, 3], [0, 1, 2, 3]):
        ids_b = np.minimum(ids, E - 2).copy()
        ids_b[0, bad] = [E + 5, -2, 77, -1][: len(bad)]
        c = (x, ids_b, w, q13, s13, q2, s2)
        print(f"[decode-head] shared={shared} dropped slots {bad}", flush=True)
        fused = _run(c, gpu, tail=True, shared_id=sid, valid_experts=E - 1 if shared else E)
        plain = _run(c, gpu, tail=False, shared_id=sid, valid_experts=E - 1 if shared else E)
        _compare(fused, plain, ids_b, E - 1 if shared else E, shared)
        assert fused[1]["invalid"] == plain[1]["invalid"] == len(bad)


@pytest.mark.parametrize("T", [1, 2])
def test_decode_shared_expert_only(gpu, T):
    """top_k = 0 with a shared expert: no ids at all (the pointers are NULL)."""
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(40 + T, T, 256, 128, 3, 1)
    ids0 = np.zeros((T, 0), np.int64)
    w0 = np.zeros((T, 0), np.float32)
    c = (x, ids0, w0, q13, s13, q2, s2)
    print(f"[decode] shared expert only, T={T}", flush=True)
    fused = _run(c, gpu, tail=True, shared_id=2)
    plain = _run(c, gpu, tail=False, shared_id=2)
    _compare(fused, plain, ids0, 3, True)
    assert fused[1]["invalid"] == plain[1]["invalid"] == 0


def test_decode_tail_repeated_expert(gpu, oracle_lib):
    """Two tokens whose ids repeat one expert: 22 routes of expert 0 (two 16-row
    blocks, the second mixing both tokens) plus the shared pair, through the tail
    and the unfused path."""
    E = 6
    x, _, _, q13, s13, q2, s2 = H.w8a8_case(50, 2, 256, 64, E, 4)
    ids = np.array([[0] * 12, [0, 0, 0, 0, 1, 2] + [0] * 6], np.int64)
    w = np.random.default_rng(51).uniform(0.05, 0.3, size=ids.shape).astype(np.float32)
    c = (x, ids, w, q13, s13, q2, s2)
    print("[decode-tail] repeated expert, T=2", flush=True)
    fused = _run(c, gpu, tail=True, shared_id=E - 1)
    plain = _run(c, gpu, tail=False, shared_id=E - 1)
    _compare(fused, plain, ids, E, True)
    ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=E - 1)
    np.testing.assert_array_equal(fused[0], ref)


def test_decode_tail_int32_ids_and_third_token_falls_back(gpu, oracle_lib):
    """int32 ids through the tail; T=3 runs the unfused path (same result)."""
    for T in (2, 3):
        case = H.w8a8_case(20 + T, T, 256, 64, 9, 2)
        x, ids, w, q13, s13, q2, s2 = case
        ids = np.minimum(ids, 7)
        case = (x, ids, w, q13, s13, q2, s2)
        fused = _run(case, gpu, tail=True, shared_id=8, ids_i64=False)
        plain = _run(case, gpu, tail=False, shared_id=8, ids_i64=False)
        _compare(fused, plain, ids, 9, True)
        ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=8)
        np.testing.assert_array_equal(fused[0], ref)
