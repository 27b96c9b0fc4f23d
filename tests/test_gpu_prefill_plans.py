"""The two W8A8 prefill launch plans (classic per-class launches side by side,
or the mixed plan: a persistent MFMA launch sharing every CU with a
persistent 16-row streaming launch) give the same bits on the same input,
and match the CPU oracle. The plan is normally chosen on the device from the
route scan's tile counts; FCMOE_PREFILL_MIXED_MIN_TILES forces it. The
classic plan may run partitioned (the 256-row class on a persistent launch
over part of the CUs, the other classes on the rest); FCMOE_PREFILL_PART=0
turns that off.
Reference semantics: csrc/moe/arm/i8mm_w8a8/kernels.cpp:463-694."""

from __future__ import annotations

import os

import numpy as np
import pytest

from tests.helpers import gpu_w8a8_forward, pack_gpu, w8a8_case

pytestmark = pytest.mark.gpu


def _run_plan(min_tiles: str, *args, part: str = "1", **kw):
    env = {"FCMOE_PREFILL_MIXED_MIN_TILES": min_tiles, "FCMOE_PREFILL_PART": part}
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return gpu_w8a8_forward(*args, **kw)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.mark.parametrize("skew", [1.2, None])
def test_prefill_plans_agree_bit_exact(gpu, oracle_lib, skew):
    # 24 routed experts + shared, 640 tokens: every class of the prefill set
    # (with Zipf skew: experts of <= 16 rows beside ones of several hundred;
    # the shared expert spans three 256-row tiles).
    H, I, E, k, T = 1024, 512, 24, 6, 640
    x, ids, w, q13, s13, q2, s2 = w8a8_case(777, T, H, I, E + 1, k, skew=skew)
    ids = np.minimum(ids, E - 1)
    packed = (pack_gpu(q13, 2, gpu), pack_gpu(q2, 1, gpu))
    counts = np.bincount(ids.ravel(), minlength=E)
    print(f"[plans] skew={skew} expert rows: min {counts.min()} max {counts.max()}", flush=True)
    args = (x, ids, w, q13, s13, q2, s2, gpu)
    kw = dict(shared_id=E, scale=2.5, packed=packed)
    mixed = _run_plan("0", *args, **kw)
    classic = _run_plan("1000000000", *args, **kw)  # partitioned when the class counts call for it
    unpart = _run_plan("1000000000", *args, part="0", **kw)
    assert np.array_equal(mixed, classic), f"{(mixed != classic).sum()} outputs differ between the plans"
    assert np.array_equal(unpart, classic), f"{(unpart != classic).sum()} outputs differ with the partition"
    tok = np.array([0, 1, T // 2, T - 1])
    ref = oracle_lib.w8a8_forward(x[tok], ids[tok], w[tok], q13, s13, q2, s2, shared_id=E, routed_scale=2.5)
    assert np.array_equal(mixed[tok], ref)
