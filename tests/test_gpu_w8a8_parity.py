"""GPU parity of the W8A8 hot path against the CPU oracle, through the C ABI.

Bar: bit-exact. Routing indices, int8 activations/scales and the int32 GEMM
accumulators are integer data; the W8A8 epilogues follow the reference's
binary32 operation sequence (FEXPA exp included) on both sides, so the bf16
outputs are compared bit for bit as well.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import helpers as H

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ route --

@pytest.mark.parametrize(
    "tokens,top_k,experts,shared,i64",
    [(1, 1, 1, False, True), (37, 2, 4, False, False), (64, 8, 257, True, True), (513, 6, 33, True, False),
     (4096, 8, 257, True, True),
     # the single-workgroup path serves up to 1024 routes, the chunked one beyond
     (128, 8, 9, False, True), (114, 8, 1024, True, False), (103, 10, 1000, False, True)],
)
def test_route_build_matches_oracle(gpu, oracle_lib, tokens, top_k, experts, shared, i64):
    rng = np.random.default_rng(tokens * 31 + experts)
    routed = experts - 1 if shared else experts
    ids = np.stack([rng.permutation(routed)[:top_k] if routed >= top_k else rng.integers(0, routed, top_k)
                    for _ in range(tokens)]).astype(np.int64)
    sid = experts - 1 if shared else -1
    c, o, s, bad = H.gpu_route_build(ids, experts, sid, gpu, ids_i64=i64)
    rc, ro, rs, rbad = oracle_lib.route_build(ids, experts, sid)
    assert bad == rbad == 0
    np.testing.assert_array_equal(c, rc)
    np.testing.assert_array_equal(o, ro)
    np.testing.assert_array_equal(s[: ro[-1]], rs)


def test_route_build_skewed_and_invalid(gpu, oracle_lib):
    rng = np.random.default_rng(5)
    ids, _ = H.zipf_topk(rng, 4096, 256, 8, s=1.2, tau=0.25)
    ids[7, 3] = 300  # out of range: counted, not placed
    ids[100, 0] = -1
    c, o, s, bad = H.gpu_route_build(ids, 257, 256, gpu)
    rc, ro, rs, rbad = oracle_lib.route_build(ids, 257, 256)
    # the oracle counts both; the GPU counts routed ids outside [0, 257)
    assert bad == 2 and rbad == 2
    np.testing.assert_array_equal(c, rc)
    np.testing.assert_array_equal(o, ro)
    np.testing.assert_array_equal(s[: ro[-1]], rs)
    assert (c == 0).sum() > 0  # skew leaves experts without tokens


def test_route_build_small_with_invalid_ids(gpu, oracle_lib):
    """Decode-sized routing (one workgroup) with out-of-range and negative ids."""
    rng = np.random.default_rng(11)
    ids = np.stack([rng.permutation(256)[:8] for _ in range(64)]).astype(np.int64)
    ids[3, 2] = 999
    ids[40, 7] = -5
    c, o, s, bad = H.gpu_route_build(ids, 257, 256, gpu)
    rc, ro, rs, rbad = oracle_lib.route_build(ids, 257, 256)
    assert bad == rbad == 2
    np.testing.assert_array_equal(c, rc)
    np.testing.assert_array_equal(o, ro)
    np.testing.assert_array_equal(s[: ro[-1]], rs)


# ------------------------------------------------------------------ quant --

@pytest.mark.parametrize("rows,cols,ldq", [(1, 16, 64), (7, 7168, 7168), (33, 2048, 2048), (5, 96, 128)])
def test_quant_rows_half_away_matches_oracle(gpu, oracle_lib, rows, cols, ldq):
    rng = np.random.default_rng(rows + cols)
    x = H.bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32) * 3)
    x[0, :] = 0  # all-zero row: scale 1, q 0
    q, s = H.gpu_quant_rows(x, 0, gpu, ldq)
    rq, rs = oracle_lib.quant_rows_away(x)
    np.testing.assert_array_equal(q[:, :cols], rq)
    assert (q[:, cols:] == 0).all()
    np.testing.assert_array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("f32", [False, True])
def test_quant_rows_ties_to_even_matches_oracle(gpu, oracle_lib, f32):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((9, 31)).astype(np.float32)
    x[1, :5] = [127.0, 0.5, 1.5, -0.5, -1.5]  # exact ties (tests/test_deepseek_v4_w8a8.py:40-50)
    x[1, 5:] = 0
    xin = x if f32 else H.bf16_bits(x)
    q, s = H.gpu_quant_rows(xin, 1, gpu, 64)
    rq, rs = oracle_lib.quant_rows_even(xin)
    np.testing.assert_array_equal(q[:, :31], rq)
    np.testing.assert_array_equal(s.view(np.uint32), rs.view(np.uint32))
    assert list(q[1, :5]) == [127, 0, 2, 0, -2]


# ----------------------------------------------------- grouped int8 GEMM --

@pytest.mark.parametrize(
    "counts,k,n",
    [
        ([1, 0, 3, 16, 17], 64, 48),            # BM 16 / 32 classes, N not a multiple of 64
        ([33, 64, 65, 128], 128, 64),           # BM 64 / 128
        ([129, 256, 600, 0, 2], 192, 80),       # BM 192 / 256 and a multi-tile expert
        ([150, 193, 7, 0, 64], 128, 48),        # BM 192 edges
        ([5, 2, 300], 7168, 64),                # DSv3 hidden as K
    ],
)
def test_grouped_gemm_int32_accumulators_exact(gpu, oracle_lib, counts, k, n):
    rng = np.random.default_rng(sum(counts) + k)
    counts = np.asarray(counts, np.int32)
    total = int(counts.sum())
    a_rows = total + 3
    a = rng.integers(-127, 128, size=(a_rows, k), dtype=np.int8)
    a[0, :] = 127  # extreme magnitudes
    row_map = rng.integers(0, a_rows, size=total).astype(np.int32)
    w = rng.integers(-127, 128, size=(len(counts), n, k), dtype=np.int8)
    w[0, 0, :] = -128
    acc, offsets = H.gpu_grouped_gemm_acc(a, row_map, counts, w, gpu)
    for e in range(len(counts)):
        lo, hi = offsets[e], offsets[e + 1]
        if hi == lo:
            continue
        ref = oracle_lib.gemm_i8_rows(a, row_map[lo:hi].astype(np.int64), w[e])
        np.testing.assert_array_equal(acc[lo:hi], ref)


# ------------------------------------------------------------ W8A8 e2e --

def _check_w8a8(gpu, oracle_lib, case, *, shared: bool, scale: float = 1.0, ids_i64: bool = True):
    x, ids, w, q13, s13, q2, s2 = case
    sid = q13.shape[0] - 1 if shared else -1
    if shared:
        ids = np.minimum(ids, q13.shape[0] - 2)
    out, st = H.gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, gpu, shared_id=sid, scale=scale, ids_i64=ids_i64,
                                 stages=True)
    ref, d = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=sid, routed_scale=scale, dumps=True)
    # stage buffers are indexed by sorted position; map them back to flat routes
    pos_route = st["sorted_routes"]
    nvalid = len(pos_route)
    np.testing.assert_array_equal(st["y"][:nvalid], d["y"][pos_route])
    np.testing.assert_array_equal(st["q2"][:nvalid], d["q2"][pos_route])
    np.testing.assert_array_equal(st["s2row"][:nvalid].view(np.uint32), d["s2row"][pos_route].view(np.uint32))
    np.testing.assert_array_equal(st["route_out"].view(np.uint32), d["route_out"].view(np.uint32))
    np.testing.assert_array_equal(out, ref)
    return out


@pytest.mark.parametrize("experts,top_k,tokens", [(1, 1, 48), (2, 1, 48), (8, 2, 32), (5, 3, 70)])
def test_w8a8_forward_bit_exact_small(gpu, oracle_lib, experts, top_k, tokens):
    # the shapes of tests/test_moe_w8a8.py:197-226 and a few multi-slot ones
    case = H.w8a8_case(100 + experts * 7 + top_k, tokens, 64, 64, experts, top_k, int_range=12)
    _check_w8a8(gpu, oracle_lib, case, shared=False)


def test_w8a8_forward_bit_exact_routed_shared(gpu, oracle_lib):
    case = H.w8a8_case(7, 32, 1024, 512, 9, 2)
    _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5, ids_i64=False)


def test_w8a8_forward_bit_exact_dsv3_hidden(gpu, oracle_lib):
    """Full DeepSeek-V3 H and F with 32 routed experts + shared, T=64, top-8."""
    case = H.w8a8_case(3, 64, 7168, 2048, 33, 8)
    _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5)


def test_w8a8_forward_bit_exact_skewed_prefill(gpu, oracle_lib):
    """Zipf-skewed routing over 64 experts: every tile class, empty experts."""
    case = H.w8a8_case(9, 1024, 256, 128, 65, 8, skew=1.2)
    _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5)


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k,skew", [
    (5, 48, 16, 4, 2, None),         # smallest legal dims (multiples of 16), K padded to 64
    (600, 208, 80, 9, 4, 1.2),       # ragged K on every tile class, the LDS kernel included
    (333, 1040, 272, 17, 6, 1.1),    # K = 1040 / 272: padded tail chunk after full ones
])
def test_w8a8_forward_bit_exact_ragged_dims(gpu, oracle_lib, tokens, hidden, inter, experts, top_k, skew):
    """H and F multiples of 16 but not of 64 (the reference's W8A8 domain,
    csrc/moe/arm/i8mm_w8a8/kernels.cpp:485-570): the packed K chunks and the
    quantised activation rows carry zero padding that must not change a bit."""
    case = H.w8a8_case(500 + hidden + inter, tokens, hidden, inter, experts + 1, top_k, skew=skew)
    _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5)


def test_w8a8_forward_repeat_bitwise(gpu, oracle_lib):
    case = H.w8a8_case(13, 40, 256, 128, 6, 2)
    x, ids, w, q13, s13, q2, s2 = case
    a = H.gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, gpu)
    b = H.gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, gpu)
    np.testing.assert_array_equal(a, b)


def test_w8a8_forward_bit_exact_odd_chunk_counts(gpu, oracle_lib):
    """K = 1040 / 272 (17 / 5 chunks of 64 bytes): the LDS-staged kernel loads
    A two chunks at a time, so its last A stage lies half past K; the 600- and
    256-row experts run the 256-row tiles (W13 on 4-wave workgroups, W2 and
    the raw-accumulator GEMM on 8-wave ones) on it."""
    case = H.w8a8_case(61, 1200, 1040, 272, 9, 4, skew=1.2)
    _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5)
    counts = np.asarray([129, 256, 600, 0, 2], np.int32)
    rng = np.random.default_rng(5)
    total = int(counts.sum())
    a = rng.integers(-127, 128, size=(total + 3, 1088), dtype=np.int8)
    row_map = rng.integers(0, total + 3, size=total).astype(np.int32)
    w = rng.integers(-127, 128, size=(len(counts), 112, 1088), dtype=np.int8)
    acc, offsets = H.gpu_grouped_gemm_acc(a, row_map, counts, w, gpu)
    for e in range(len(counts)):
        lo, hi = offsets[e], offsets[e + 1]
        if hi > lo:
            np.testing.assert_array_equal(acc[lo:hi], oracle_lib.gemm_i8_rows(a, row_map[lo:hi].astype(np.int64), w[e]))


@pytest.mark.parametrize("tokens", [128, 129])
def test_w8a8_forward_bit_exact_route_path_boundary(gpu, oracle_lib, tokens):
    """1024 routes (128 tokens x top-8) is the largest routing the single-
    workgroup route kernel takes, and there the token rows are quantised in
    the same launch (32 groups of 4 rows); 129 tokens (1032 routes) take the
    count / scan / scatter kernels and the separate row quantisation."""
    case = H.w8a8_case(900 + tokens, tokens, 512, 256, 16, 8)
    _check_w8a8(gpu, oracle_lib, case, shared=False)


@pytest.mark.parametrize("tokens", [1, 2, 5])
def test_w8a8_forward_bit_exact_small_batch(gpu, oracle_lib, tokens):
    """Small-batch decode (1-5 tokens, 4 routed experts each plus the shared
    one): one-row tiles, most tile rows padding. Bit-exact against
    the oracle, and repeatable across two calls."""
    case = H.w8a8_case(700 + tokens, tokens, 4096, 2048, 17, 4)
    a = _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5)
    b = _check_w8a8(gpu, oracle_lib, case, shared=True, scale=2.5)
    np.testing.assert_array_equal(a, b)
