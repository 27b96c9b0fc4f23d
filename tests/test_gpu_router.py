"""GPU top-k softmax router (``fcmoe_router_topk`` via ``fused_cpp_amd.router``)
against the CPU oracle's closed form.

Bar: ids bit-exact (descending logit order, lower id on ties); weights within
rtol 4e-6 (the kernel's expf and its butterfly sum order against numpy's exp
and pairwise sum: a few fp32 ulps).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

RTOL = 4e-6


def _run(x, k, **kw):
    from fused_cpp_amd import router

    ids, w = router.topk_softmax(torch.from_numpy(x).cuda(), k, **kw)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("tokens,experts,k,scale", [(32, 8, 2, 1.0), (64, 256, 8, 2.5), (4096, 256, 8, 2.5),
                                                     (8192, 384, 8, 2.5), (3, 1024, 64, 1.0), (9, 5, 5, 1.0),
                                                     (17, 100, 7, 1.0)])
def test_router_matches_oracle(gpu, oracle_lib, tokens, experts, k, scale):
    rng = np.random.default_rng(tokens + experts)
    x = rng.standard_normal((tokens, experts)).astype(np.float32)
    ids, w = _run(x, k, scale=scale)
    rids, rw = oracle_lib.router_topk(x, k, scale=scale)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_allclose(w, rw, rtol=RTOL, atol=1e-9)


def test_router_int32_ids_no_renorm(gpu, oracle_lib):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((50, 64)) * 4).astype(np.float32)
    ids, w = _run(x, 6, renormalize=False, ids_dtype=torch.int32)
    rids, rw = oracle_lib.router_topk(x, 6, renormalize=False)
    assert ids.dtype == np.int32
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_allclose(w, rw, rtol=RTOL, atol=1e-9)


def test_router_ties_and_infinities(gpu, oracle_lib):
    x = np.zeros((4, 70), np.float32)
    x[1, [3, 66, 9]] = 2.0          # equal maxima across lanes and lane rounds
    x[2, :] = -np.inf
    x[2, [5, 40]] = [1.0, 0.5]      # fewer finite logits than k
    x[3, :] = np.arange(70, dtype=np.float32)[::-1]
    ids, w = _run(x, 3)
    assert ids[0].tolist() == [0, 1, 2]
    assert ids[1].tolist() == [3, 9, 66]
    # fewer finite logits than k: the rest in id order, never a repeated id
    assert ids[2].tolist() == [5, 40, 0]
    assert ids[3].tolist() == [0, 1, 2]
    np.testing.assert_array_equal(ids, oracle_lib.router_topk(x, 3)[0])
    for row in ids:
        assert len(set(row.tolist())) == 3
    np.testing.assert_allclose(w[[0, 1, 3]], oracle_lib.router_topk(x[[0, 1, 3]], 3)[1], rtol=RTOL)
    np.testing.assert_allclose(w[2].sum(), 1.0, rtol=1e-6)


def test_router_ids_distinct_with_infinities_and_nans(gpu, oracle_lib):
    """One finite logit and k = 2, or NaNs only: ids stay distinct (an expert
    already chosen never wins a later round) and follow the oracle's order
    (NaN logits rank last, lower id first)."""
    x = np.full((3, 4), -np.inf, np.float32)
    x[0, 0] = 1.0                      # [1, -inf, -inf, -inf], k = 2
    x[1, :] = np.nan
    x[2, :] = [np.nan, 0.5, np.nan, -np.inf]
    ids, w = _run(x, 2)
    assert ids[0].tolist() == [0, 1]
    assert ids[1].tolist() == [0, 1]
    assert ids[2].tolist() == [1, 3]
    np.testing.assert_array_equal(ids, oracle_lib.router_topk(x, 2)[0])
    np.testing.assert_allclose(w[0], [1.0, 0.0], rtol=1e-6)


def test_router_feeds_w8a8_forward(gpu):
    """GPU router output drives the fused op unchanged (ids int64, weights fp32)."""
    from fused_cpp_amd import router

    rng = np.random.default_rng(0)
    ids, w = router.topk_softmax(torch.from_numpy(rng.standard_normal((16, 32)).astype(np.float32)).cuda(), 4,
                                 scale=2.5)
    torch.cuda.synchronize()
    assert ids.dtype == torch.int64 and w.dtype == torch.float32 and ids.shape == (16, 4)
    assert int(ids.min()) >= 0 and int(ids.max()) < 32
    np.testing.assert_allclose(w.sum(dim=1).cpu().numpy(), 2.5, rtol=1e-6)


def test_router_rejects_bad_args(gpu):
    from fused_cpp_amd import router

    x = torch.zeros((4, 8), device="cuda")
    with pytest.raises(ValueError):
        router.topk_softmax(x, 9)
    with pytest.raises(TypeError):
        router.topk_softmax(x.double(), 2)
    ids, w = router.topk_softmax(torch.zeros((0, 8), device="cuda"), 2)
    assert ids.shape == (0, 2)
