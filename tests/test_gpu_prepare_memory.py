"""Routed + shared prepare packs the shared expert straight into the routed
experts' buffer: the packed bytes equal those of packing the concatenated
[E + 1] weights, and the device never holds a second (concatenated) copy of
the weights -- peak device memory added during prepare stays within 1.1x the
packed size, for host sources (staged a chunk at a time) and for device
sources (the caller's own tensors aside). Reference: the routed+shared
prepares of src/fused_cpp/moe/bf16_tiled.py:541-609 (native
fused_moe_bf16_tiled.cpp:6276-6288) pack "without a full source copy"."""

from __future__ import annotations

import pytest
import torch

from fused_cpp_amd import moe

pytestmark = pytest.mark.gpu


def _peak_added(fn):
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - base


def _packed_bytes(*tensors):
    return sum(t.numel() * t.element_size() for t in tensors)


@pytest.mark.parametrize("on_device", [False, True])
def test_int8_routed_shared_prepare_no_second_copy(gpu, on_device):
    E, H, F = 48, 1024, 512
    g = torch.Generator().manual_seed(3)
    rw13 = torch.randint(-127, 128, (E, 2 * F, H), dtype=torch.int8, generator=g)
    rw2 = torch.randint(-127, 128, (E, H, F), dtype=torch.int8, generator=g)
    sw13 = torch.randint(-127, 128, (2 * F, H), dtype=torch.int8, generator=g)
    sw2 = torch.randint(-127, 128, (H, F), dtype=torch.int8, generator=g)
    rs13, rs2 = torch.rand(E, 2 * F, generator=g), torch.rand(E, H, generator=g)
    ss13, ss2 = torch.rand(2 * F, generator=g), torch.rand(H, generator=g)
    args = [rw13, rs13, rw2, rs2, sw13, ss13, sw2, ss2]
    if on_device:
        args = [a.to(gpu) for a in args]
    print(f"[prepare] int8 routed+shared E={E} on_device={on_device}", flush=True)
    prep, added = _peak_added(lambda: moe.prepare_routed_shared_moe_w8a8_tiled_quantized_weights(*args))
    p = prep.packed
    packed = _packed_bytes(p.w13[0], p.w13[3], p.w2[0], p.w2[3])
    assert added <= 1.1 * packed, f"prepare added {added} bytes for {packed} packed bytes"
    ref = moe.prepare_fused_moe_w8a8_tiled_quantized_weights(
        torch.cat((rw13, sw13[None])).to(gpu), torch.cat((rs13, ss13[None])).to(gpu),
        torch.cat((rw2, sw2[None])).to(gpu), torch.cat((rs2, ss2[None])).to(gpu))
    for a, b in ((p.w13[0], ref.w13[0]), (p.w13[3], ref.w13[3]), (p.w2[0], ref.w2[0]), (p.w2[3], ref.w2[3])):
        assert torch.equal(a, b)
    assert p.w13[1:3] == ref.w13[1:3] and p.w2[1:3] == ref.w2[1:3]
    w8 = moe.prepare_routed_shared_moe_w8a16_tiled_quantized_weights(*args)
    assert torch.equal(w8.packed.w13[0], ref.w13[0]) and torch.equal(w8.packed.w2[0], ref.w2[0])


@pytest.mark.parametrize("on_device", [False, True])
def test_bf16_routed_shared_prepare_no_second_copy(gpu, on_device):
    E, H, F = 24, 1024, 512
    g = torch.Generator().manual_seed(4)
    rw13 = (torch.randn(E, 2 * F, H, generator=g) * 0.02).bfloat16()
    rw2 = (torch.randn(E, H, F, generator=g) * 0.02).bfloat16()
    sw13 = (torch.randn(2 * F, H, generator=g) * 0.02).bfloat16()
    sw2 = (torch.randn(H, F, generator=g) * 0.02).bfloat16()
    args = [rw13, rw2, sw13, sw2]
    if on_device:
        args = [a.to(gpu) for a in args]
    print(f"[prepare] bf16 routed+shared E={E} on_device={on_device}", flush=True)
    prep, added = _peak_added(lambda: moe.prepare_routed_shared_moe_bf16_tiled_weights(*args))
    p = prep.packed
    packed = _packed_bytes(p.w13[0], p.w2[0])
    assert added <= 1.1 * packed, f"prepare added {added} bytes for {packed} packed bytes"
    ref = moe.prepare_fused_moe_bf16_tiled_weights(torch.cat((rw13, sw13[None])).to(gpu),
                                                   torch.cat((rw2, sw2[None])).to(gpu), fuse_silu=True)
    assert torch.equal(p.w13[0], ref.w13[0]) and torch.equal(p.w2[0], ref.w2[0])
    assert p.w13[1:] == ref.w13[1:] and p.w2[1:] == ref.w2[1:] and p.fused_silu
