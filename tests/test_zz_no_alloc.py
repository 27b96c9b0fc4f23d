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
    # 5 tokens: the single decode class.
    for tokens in (96, 5):
        print(f"[noalloc] tokens={tokens} H={H} I={I} E={E}+1 top-{k}", flush=True)
        args = (x[:tokens], ids[:tokens], w[:tokens], q13, s13, q2, s2, gpu)
        kw = dict(shared_id=E, scale=2.5, packed=packed)
        ref = gpu_w8a8_forward(*args, **kw)
        got = gpu_w8a8_forward(*args, **kw, noalloc=True)
        assert got.shape == (tokens, H)
        assert np.array_equal(got, ref), f"{(got != ref).sum()} of {got.size} outputs differ at tokens={tokens}"
