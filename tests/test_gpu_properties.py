"""Size-independent properties of the W8A8 forward at the BASELINE workloads.

Every token's output depends only on its own row, routing ids and weights:
the activation quantisation is per token row, the int8 GEMMs accumulate
exact int32 sums per row, and the merge runs over the token's own slots
(csrc/moe/arm/i8mm_w8a8/kernels.cpp:463-694). Permuting the tokens must
therefore permute the output rows bit for bit, whatever tile classes,
launch plan (classic, partitioned or mixed), row tiles and channel blocks the
permuted routing lands in. This checks every token of the full-size layers,
where the oracle comparison can only sample a few.
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_w8a8_token_permutation_equivariance(gpu, name):
    from fused_cpp_amd.moe import fused_moe_w8a8_tiled_with_shared

    cfg = bench.CONFIGS[name]
    ids, w, _ = bench.make_routing(cfg)
    x = bench.make_x(cfg, gpu)
    weights, _ = bench.build_layer(cfg, gpu, False)
    counts = bench.expert_counts(cfg, ids)
    plan = bench.prefill_plan(counts)[0] if counts.sum() > 8 * len(counts) else "decode"
    print(f"[properties] {name}: T={cfg['T']} plan {plan}", flush=True)

    def run(xx, ww, ii):
        return fused_moe_w8a8_tiled_with_shared(xx, weights, torch.from_numpy(ww).to(gpu),
                                                torch.from_numpy(ii).to(gpu), routed_scaling_factor=cfg["scale"])

    base = run(x, w, ids)
    perm = np.random.default_rng(5).permutation(cfg["T"])
    permuted = run(x[torch.from_numpy(perm).to(gpu)], np.ascontiguousarray(w[perm]), np.ascontiguousarray(ids[perm]))
    torch.cuda.synchronize()
    same = permuted.view(torch.int16) == base[torch.from_numpy(perm).to(gpu)].view(torch.int16)
    bad = (~same).any(dim=1).nonzero().flatten()
    assert bad.numel() == 0, f"{bad.numel()} permuted tokens differ, first {bad[:8].tolist()}"
    # a token repeated in place of another gets the repeated token's output
    dup = ids.copy(), w.copy()
    dup[0][1], dup[1][1] = ids[0], w[0]
    xd = x.clone()
    xd[1] = x[0]
    rep = run(xd, dup[1], dup[0])
    assert torch.equal(rep[1].view(torch.int16), base[0].view(torch.int16))
    del weights, base, permuted, rep
    gc.collect()
    torch.cuda.empty_cache()
