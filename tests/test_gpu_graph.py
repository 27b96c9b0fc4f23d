"""The fused-MoE operators under HIP graph capture (torch.cuda.CUDAGraph).

Each graph is replayed several times with new inputs copied into its static
buffers and unrelated eager work plus synchronisations between replays; every
replay must equal the eager result bit for bit (the same kernels run).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _replay_matches_eager(fn, make_inputs, static_inputs, replays=3):
    torch.cuda.synchronize()
    # warm up on a side stream (allocator pools, side streams, lazily created events)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn(*static_inputs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = fn(*static_inputs)
    for r in range(replays):
        fresh = make_inputs(r)
        for dst, src in zip(static_inputs, fresh):
            if isinstance(dst, torch.Tensor):
                dst.copy_(src)
        noise = torch.randn(4096, device=static_out.device).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        expected = fn(*fresh)
        torch.cuda.synchronize()
        assert torch.equal(static_out, expected), f"replay {r} differs from eager"
        assert torch.isfinite(noise)


def test_w8a8_forward_graph_replays(gpu):
    from fused_cpp_amd import moe

    case = H.w8a8_case(21, 48, 1024, 512, 17, 4)
    x, ids, w, q13, s13, q2, s2 = case
    t = torch.from_numpy
    prepared = moe.prepare_routed_shared_moe_w8a8_tiled_quantized_weights(
        t(q13[:-1]), t(s13[:-1]), t(q2[:-1]), t(s2[:-1]), t(q13[-1]), t(s13[-1]), t(q2[-1]), t(s2[-1]))
    ids = np.minimum(ids, 15)
    rng = np.random.default_rng(0)

    def make(r):
        xr = torch.from_numpy(H.bf16_bits(rng.standard_normal((48, 1024)).astype(np.float32)).view(np.int16))
        idr = torch.from_numpy(rng.integers(0, 16, size=(48, 4)).astype(np.int64))
        wr = torch.from_numpy(rng.random((48, 4)).astype(np.float32))
        return xr.to(gpu).view(torch.bfloat16), wr.to(gpu), idr.to(gpu)

    static = list(make(-1))

    def fn(xx, ww, ii):
        return moe.fused_moe_w8a8_tiled_with_shared(xx, prepared, ww, ii, routed_scaling_factor=2.5)

    _replay_matches_eager(fn, make, static)


def test_w8a8_one_token_decode_graph_replays(gpu):
    """One token: the decode head and tail launches (route + quantisation + W13,
    then requant + W2 + merge) under capture."""
    from fused_cpp_amd import moe

    case = H.w8a8_case(23, 1, 1024, 512, 17, 4)
    x, ids, w, q13, s13, q2, s2 = case
    t = torch.from_numpy
    prepared = moe.prepare_routed_shared_moe_w8a8_tiled_quantized_weights(
        t(q13[:-1]), t(s13[:-1]), t(q2[:-1]), t(s2[:-1]), t(q13[-1]), t(s13[-1]), t(q2[-1]), t(s2[-1]))
    rng = np.random.default_rng(5)

    def make(r):
        xr = torch.from_numpy(H.bf16_bits(rng.standard_normal((1, 1024)).astype(np.float32)).view(np.int16))
        idr = torch.from_numpy(rng.choice(16, size=(1, 4), replace=False).astype(np.int64))
        wr = torch.from_numpy(rng.random((1, 4)).astype(np.float32))
        return xr.to(gpu).view(torch.bfloat16), wr.to(gpu), idr.to(gpu)

    static = list(make(-1))

    def fn(xx, ww, ii):
        return moe.fused_moe_w8a8_tiled_with_shared(xx, prepared, ww, ii, routed_scaling_factor=2.5)

    _replay_matches_eager(fn, make, static)


def test_bf16_and_w8a16_forward_graph_replays(gpu):
    from fused_cpp_amd import moe

    rng = np.random.default_rng(3)
    T, Hd, F, E, k = 16, 512, 256, 8, 2
    w13 = H.bf16_bits((rng.standard_normal((E, 2 * F, Hd)) * 0.02).astype(np.float32))
    w2 = H.bf16_bits((rng.standard_normal((E, Hd, F)) * 0.02).astype(np.float32))
    tb = lambda b: torch.from_numpy(b.view(np.int16)).to(gpu).view(torch.bfloat16)  # noqa: E731
    bf16_w = moe.prepare_fused_moe_bf16_tiled_weights(tb(w13), tb(w2), fuse_silu=True)
    w8_w = moe.prepare_fused_moe_w8a16_tiled_weights(tb(w13), tb(w2))

    def make(r):
        xr = tb(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
        ids, w = H.softmax_topk(rng.standard_normal((T, E)).astype(np.float32), k)
        return xr, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu)

    for weights, op in ((bf16_w, moe.fused_moe_bf16_tiled), (w8_w, moe.fused_moe_w8a16_tiled)):
        static = list(make(-1))
        _replay_matches_eager(lambda xx, ww, ii: op(xx, weights, ww, ii), make, static)


@pytest.mark.parametrize("T", [1, 64, 200])
def test_bf16_shared_mlp_and_one_expert_graph_replays(gpu, T):
    """The small-M BF16 forward under capture: the dense shared MLP (no route
    build; its merge launch zeroes the invalid-id count) and a one-expert MoE
    (route build, the W2 reduce merging each token's route)."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(T)
    Hd, F = 1024, 512
    tb = lambda b: torch.from_numpy(b.view(np.int16)).to(gpu).view(torch.bfloat16)  # noqa: E731
    w13 = H.bf16_bits((rng.standard_normal((2 * F, Hd)) * 0.02).astype(np.float32))
    w2 = H.bf16_bits((rng.standard_normal((Hd, F)) * 0.02).astype(np.float32))
    sm = moe.prepare_shared_mlp_bf16_tiled_weights(tb(w13), tb(w2))
    ones = torch.ones((T, 1), device=gpu)
    zeros = torch.zeros((T, 1), dtype=torch.int32, device=gpu)

    def make(r):
        return (tb(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32))),
                torch.from_numpy(rng.random((T, 1)).astype(np.float32) + 0.5).to(gpu))

    static = list(make(-1))

    def fn(xx, ww):
        a = moe.shared_mlp_bf16_tiled(xx, sm)
        b = moe.fused_moe_bf16_tiled(xx, sm, ww, zeros)
        c = moe.fused_moe_bf16_tiled(xx, sm, ones, zeros)
        return torch.cat([a.float().reshape(-1), b.float().reshape(-1), c.float().reshape(-1)])

    _replay_matches_eager(fn, make, static)
    out = fn(*static)
    n = T * Hd
    assert torch.equal(out[:n], out[2 * n:])  # shared MLP == one-expert MoE with weight 1


def test_router_and_i8gemm_graph_replays(gpu):
    from fused_cpp_amd import i8gemm, router

    rng = np.random.default_rng(5)
    weight = torch.randint(-16, 17, (96, 256), dtype=torch.int8)
    packed = i8gemm.prepare(weight, torch.rand(96) * 0.01 + 0.001)

    def make(r):
        return (torch.randn(40, 256, device=gpu).to(torch.bfloat16),
                torch.from_numpy(rng.standard_normal((40, 64)).astype(np.float32)).to(gpu))

    static = list(make(-1))

    def fn(xx, logits):
        ids, w = router.topk_softmax(logits, 6, scale=2.5)
        out = i8gemm.dynamic_scaled_mm(xx, packed, out_dtype=torch.bfloat16)
        return torch.cat([out.float().reshape(-1), w.reshape(-1), ids.float().reshape(-1)])

    _replay_matches_eager(fn, make, static)


@pytest.mark.parametrize("m,k,n", [(64, 8192, 1000), (300, 4096, 700), (520, 256, 300)])
def test_i8gemm_split_k_graph_replays(gpu, m, k, n):
    """i8gemm and the pair with their K-split partial sums and reduce launches
    (small-M kernel at 64 rows; the LDS tiles split 4 ways at 300 rows; no
    split at 520 rows and K = 256) captured and replayed."""
    from fused_cpp_amd import i8gemm

    g = torch.Generator().manual_seed(m + k + n)
    w1 = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    w2 = torch.randint(-127, 128, (n // 2 + 3, k), dtype=torch.int8, generator=g)
    p1 = i8gemm.prepare(w1, torch.rand(n, generator=g) * 0.01 + 0.001)
    p2 = i8gemm.prepare(w2, torch.rand(n // 2 + 3, generator=g) * 0.01 + 0.001)
    bias = torch.randn(n, device=gpu)

    def make(r):
        return (torch.randn(m, k, device=gpu).to(torch.bfloat16),)

    static = list(make(-1))

    def fn(xx):
        out = i8gemm.dynamic_scaled_mm(xx, p1, bias=bias, out_dtype=torch.float32)
        a, b = i8gemm.dynamic_scaled_mm_pair(xx, p1, p2)
        return torch.cat([out.reshape(-1), a.float().reshape(-1), b.float().reshape(-1)])

    _replay_matches_eager(fn, make, static)


@pytest.mark.parametrize("min_tiles", ["32", "0", "1000000"])
def test_w8a8_prefill_mixed_plan_graph_replays(gpu, min_tiles):
    """Skewed prefill routing where the device picks the mixed launch plan
    (persistent MFMA launch beside the 16-row streaming launch, forked streams,
    per-XCD work queues zeroed by the route launch): "32" (the default) enqueues
    both plans (the classic launches exit on the device), "0" forces the mixed
    plan alone, "1000000" the classic plan, here partitioned (the persistent
    launch runs the 256-row class on part of the CUs beside the classic
    launches of the other classes)."""
    import os

    from fused_cpp_amd import moe

    T, Hd, F, E, k = 2048, 1024, 512, 160, 6
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(31, T, Hd, F, E + 1, k, skew=1.2)
    ids = np.minimum(ids, E - 1)
    t = torch.from_numpy
    prepared = moe.prepare_routed_shared_moe_w8a8_tiled_quantized_weights(
        t(q13[:-1]), t(s13[:-1]), t(q2[:-1]), t(s2[:-1]), t(q13[-1]), t(s13[-1]), t(q2[-1]), t(s2[-1]))
    counts = np.bincount(ids.ravel(), minlength=E)
    # the mixed plan's default trigger: >= 32 tiles of <= 16 rows, >= 16 tiles of 256 rows
    assert ((counts > 0) & (counts <= 16)).sum() >= 32, counts
    assert sum((int(c) + 255) // 256 for c in counts if c > 192) + (T + 255) // 256 >= 16, counts
    if min_tiles == "1000000":
        from fused_cpp_amd import cabi

        allc = np.append(counts, T)  # the shared expert takes every token
        tiles = [int(((allc > 0) & (allc <= 16)).sum()), int(((allc > 16) & (allc <= 128)).sum()),
                 int(((allc > 128) & (allc <= 192)).sum()), int(sum((int(c) + 255) // 256 for c in allc if c > 192))]
        saved = os.environ.get("FCMOE_PREFILL_MIXED_MIN_TILES")
        os.environ["FCMOE_PREFILL_MIXED_MIN_TILES"] = min_tiles
        try:
            assert cabi.w8a8_prefill_plan(tiles)[0] == "partitioned", tiles
        finally:
            if saved is None:
                del os.environ["FCMOE_PREFILL_MIXED_MIN_TILES"]
            else:
                os.environ["FCMOE_PREFILL_MIXED_MIN_TILES"] = saved
    rng = np.random.default_rng(1)

    def make(r):
        xr = torch.from_numpy(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)).view(np.int16))
        _, wr = H.zipf_topk(rng, T, E, k)
        return xr.to(gpu).view(torch.bfloat16), torch.from_numpy(wr).to(gpu), torch.from_numpy(ids).to(gpu)

    static = list(make(-1))

    def fn(xx, ww, ii):
        return moe.fused_moe_w8a8_tiled_with_shared(xx, prepared, ww, ii, routed_scaling_factor=2.5)

    old = os.environ.get("FCMOE_PREFILL_MIXED_MIN_TILES")
    os.environ["FCMOE_PREFILL_MIXED_MIN_TILES"] = min_tiles
    try:
        _replay_matches_eager(fn, make, static)
    finally:
        if old is None:
            del os.environ["FCMOE_PREFILL_MIXED_MIN_TILES"]
        else:
            os.environ["FCMOE_PREFILL_MIXED_MIN_TILES"] = old


def test_side_to_side_stream_wait_refused_under_capture(gpu):
    """The prefill fork joins side streams only through the caller's stream;
    a wait of one side stream on another's event (FCMOE_SIDE_CHAIN_WAIT=1 adds
    one) runs eagerly, bit-exact with the default fork, and is refused under
    graph capture before the forward enqueues anything (the capture then ends
    empty and replays nothing)."""
    import os

    from fused_cpp_amd import moe

    T, Hd, F, E, k = 2048, 1024, 512, 160, 6
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(31, T, Hd, F, E + 1, k, skew=1.2)
    ids = np.minimum(ids, E - 1)
    t = torch.from_numpy
    prepared = moe.prepare_routed_shared_moe_w8a8_tiled_quantized_weights(
        t(q13[:-1]), t(s13[:-1]), t(q2[:-1]), t(s2[:-1]), t(q13[-1]), t(s13[-1]), t(q2[-1]), t(s2[-1]))
    xd = torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.bfloat16)
    wd, idd = torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu)

    def fn(out=None):
        return moe.fused_moe_w8a8_tiled_with_shared(xd, prepared, wd, idd, routed_scaling_factor=2.5, out=out)

    ref = fn()
    torch.cuda.synchronize()
    old = os.environ.get("FCMOE_SIDE_CHAIN_WAIT")
    os.environ["FCMOE_SIDE_CHAIN_WAIT"] = "1"
    try:
        chained = fn()
        torch.cuda.synchronize()
        assert torch.equal(chained, ref)
        static = torch.zeros_like(ref)
        g = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="refused under HIP graph capture"):
            with torch.cuda.graph(g):
                fn(out=static)
        torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ["FCMOE_SIDE_CHAIN_WAIT"]
        else:
            os.environ["FCMOE_SIDE_CHAIN_WAIT"] = old
    # nothing was captured: the output buffer is untouched, and the default
    # fork still captures and replays
    assert not static.any()
    g2 = torch.cuda.CUDAGraph()
    static2 = torch.zeros_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(out=static2)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g2):
        fn(out=static2)
    static2.zero_()
    g2.replay()
    torch.cuda.synchronize()
    assert torch.equal(static2, ref)
