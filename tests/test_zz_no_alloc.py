"""fcmoe_w8a8_forward_noalloc (the entry point that allocates nothing: its
workspace is a fixed per-GPU device array) against fcmoe_w8a8_forward on the
same inputs, bit for bit, on two calls in a row -- the second one smaller, so
that a stale value the first call left in the shared array would show."""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import gpu_w8a8_forward, pack_gpu, w8a8_case

pytestmark = pytest.mark.gpu


def test_noalloc_matches_workspace_forward_on_two_calls(gpu):
    H, I, E, k = 1024, 512, 16, 8
    x, ids, w, q13, s13, q2, s2 = w8a8_case(4242, 96, H, I, E + 1, k)
    ids = np.minimum(ids, E - 1)  # routed ids stay below the shared slot
    packed = (pack_gpu(q13, 2, gpu), pack_gpu(q2, 1, gpu))
    # 96 tokens: several prefill tile classes (run in order on one stream);
    # 5 tokens: the single decode class; 1 token: the decode head and tail launches.
    for tokens in (96, 5, 1):
        print(f"[noalloc] tokens={tokens} H={H} I={I} E={E}+1 top-{k}", flush=True)
        args = (x[:tokens], ids[:tokens], w[:tokens], q13, s13, q2, s2, gpu)
        kw = dict(shared_id=E, scale=2.5, packed=packed)
        ref = gpu_w8a8_forward(*args, **kw)
        got = gpu_w8a8_forward(*args, **kw, noalloc=True)
        assert got.shape == (tokens, H)
        assert np.array_equal(got, ref), f"{(got != ref).sum()} of {got.size} outputs differ at tokens={tokens}"


def test_noalloc_graph_capture_replays_match_workspace_forward(gpu):
    """The no-alloc forward captured into a HIP graph (its intended caller):
    each replay, with new token rows and routing copied into the static
    inputs and eager work between replays, equals the workspace forward bit
    for bit. 24 tokens (one decode class) and 1 token (the decode head and
    tail launches)."""
    import ctypes

    import torch

    from fused_cpp_amd import cabi
    from tests.helpers import bf16_bits

    H, I, E, k = 1024, 512, 16, 8
    _, _, _, q13, s13, q2, s2 = w8a8_case(777, 4, H, I, E + 1, k)
    packed = (pack_gpu(q13, 2, gpu), pack_gpu(q2, 1, gpu))
    s13t, s2t = torch.from_numpy(s13).to(gpu), torch.from_numpy(s2).to(gpu)
    rng = np.random.default_rng(9)
    L = cabi.lib()
    for tokens in (24, 1):
        print(f"[noalloc-graph] tokens={tokens} H={H} I={I} E={E}+1 top-{k}", flush=True)

        def make():
            x = bf16_bits(rng.standard_normal((tokens, H)).astype(np.float32))
            ids = np.stack([rng.choice(E, k, replace=False) for _ in range(tokens)]).astype(np.int64)
            w = rng.random((tokens, k)).astype(np.float32)
            return x, ids, w

        x0, ids0, w0 = make()
        xs = torch.from_numpy(x0.view(np.int16)).to(gpu)
        idss = torch.from_numpy(ids0).to(gpu)
        ws = torch.from_numpy(w0).to(gpu)
        out = torch.zeros((tokens, H), dtype=torch.int16, device=gpu)
        inv = torch.zeros(1, dtype=torch.int32, device=gpu)
        a = cabi.MoeArgs()
        a.x, a.tokens, a.hidden, a.inter = xs.data_ptr(), tokens, H, I
        a.topk_ids, a.ids_is_i64, a.topk_weights, a.top_k = idss.data_ptr(), 1, ws.data_ptr(), k
        a.experts, a.valid_experts, a.shared_expert_id, a.routed_scaling = E + 1, E + 1, E, 2.5
        a.w13, a.w2 = packed[0].data_ptr(), packed[1].data_ptr()
        a.w13_scale, a.w2_scale = s13t.data_ptr(), s2t.data_ptr()
        a.activation = cabi.FCMOE_ACT_SILU_CLAMP10
        a.out, a.invalid_count = out.data_ptr(), inv.data_ptr()

        def call():
            cabi.check(L.fcmoe_w8a8_forward_noalloc(ctypes.byref(a), cabi.stream_handle()), "w8a8_forward_noalloc")

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            call()  # first call on the device: the scratch address is looked up outside the capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
        for r in range(3):
            x, ids, w = make()
            xs.copy_(torch.from_numpy(x.view(np.int16)))
            idss.copy_(torch.from_numpy(ids))
            ws.copy_(torch.from_numpy(w))
            noise = torch.randn(4096, device=gpu).sum()
            g.replay()
            torch.cuda.synchronize()
            got = out.cpu().numpy().view(np.uint16)
            ref = gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, gpu, shared_id=E, scale=2.5, packed=packed)
            assert np.array_equal(got, ref), f"replay {r}: {(got != ref).sum()} outputs differ (tokens={tokens})"
            assert torch.isfinite(noise)
