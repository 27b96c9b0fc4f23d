"""The BF16 top-k merge, bit for bit against the oracle's restatement of
csrc/moe/arm/sve_bf16/route_merge.cpp:38-126 on the kernel's own route rows.

The GEMMs of the BF16 path are held to tolerance (their accumulation order is
the SVE BFMMLA's, which is not restated), but the merge that follows them is
deterministic: given the fp32 route rows the W2 stage wrote and the combined
weights, the output bits are fixed -- a power-of-two split tree of weighted
leaves for top-k (with the shared slot) in {2, 4, 6, 8}, an ordered fused
multiply-add chain otherwise. A wrong tree or a wrong order fails here.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _case(seed, T, Hd, F, E, k):
    rng = np.random.default_rng(seed)
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, 2 * F, Hd)) * 0.05).astype(np.float32)))
    w2 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, Hd, F)) * 0.05).astype(np.float32)))
    ids, w = H.softmax_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    return x, w13, w2, ids, w


@pytest.mark.parametrize("top_k,shared", [(2, False), (4, False), (5, True), (6, False), (8, False), (8, True),
                                          (5, False), (9, False), (3, True)])
def test_bf16_merge_bit_exact(gpu, oracle_lib, top_k, shared):
    E = 10
    x, w13, w2, ids, w = _case(70 + top_k, 37, 320, 96, E + (1 if shared else 0), top_k)
    ids = ids % E
    # distinct ids per token after the modulo: re-draw rows that collide
    for t in range(ids.shape[0]):
        ids[t] = np.random.default_rng(t).permutation(E)[:top_k]
    out, pos, rw, route_out = H.gpu_bf16_forward(x, ids, w, w13, w2, gpu, shared_id=E if shared else -1,
                                                 scale=2.5 if shared else 1.0)
    kt = top_k + (1 if shared else 0)
    assert (pos >= 0).all()
    # the combined weights are the routing weights (x scale), shared slot 1.0
    want_w = np.concatenate([w * np.float32(2.5), np.ones((len(w), 1), np.float32)], 1) if shared else w
    np.testing.assert_array_equal(rw, want_w.reshape(-1).astype(np.float32))
    np.testing.assert_array_equal(out, oracle_lib.bf16_route_merge(route_out, rw, kt))


@pytest.mark.parametrize("top_k", [8, 5])
def test_bf16_merge_drops_invalid_route_with_validation_off(gpu, oracle_lib, top_k):
    """An out-of-range id (ids are not checked on the host here) drops its
    route: it contributes nothing, in the tree merge (top_k 8) and in the
    ordered chain (top_k 5), whatever the unwritten row holds."""
    E = 12
    x, w13, w2, ids, w = _case(90 + top_k, 21, 256, 64, E, top_k)
    for t in range(ids.shape[0]):
        ids[t] = np.random.default_rng(100 + t).permutation(E)[:top_k]
    ids[3, 2] = E + 3
    ids[7, 0] = 10 ** 6
    out, pos, rw, route_out = H.gpu_bf16_forward(x, ids, w, w13, w2, gpu, valid_experts=E)
    dropped = pos < 0
    assert dropped.sum() == 2 and dropped[3 * top_k + 2] and dropped[7 * top_k]
    rows = route_out.copy()
    wts = rw.copy()
    rows[dropped] = 0.0  # a dropped leaf is exactly 0
    wts[dropped] = 0.0
    ref = oracle_lib.bf16_route_merge(rows, wts, top_k)
    np.testing.assert_array_equal(out, ref)
    assert np.isfinite(H.bits_to_f32(out)).all()
