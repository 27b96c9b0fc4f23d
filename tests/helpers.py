"""Seeded case generators and C-ABI runners shared by the tests."""

from __future__ import annotations

import ctypes

import numpy as np

# ---------------------------------------------------------------- inputs --


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (nearest even) and return the uint16 bit patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    lsb = (u >> 16) & 1
    return ((u + np.uint32(0x7FFF) + lsb) >> 16).astype(np.uint16)


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_half_ulp(x: np.ndarray) -> np.ndarray:
    """Half a bf16 ulp at each |x| (8 significant bits): the rounding error a
    correctly rounded bf16 output already carries against an fp32 reference.
    At |x| >= 8 it is 2^-5 = 0.031, above a 2e-2 absolute bound."""
    _, e = np.frexp(np.abs(np.asarray(x, np.float64)))
    return np.ldexp(1.0, e - 9)


def softmax_topk(logits: np.ndarray, k: int, scale: float = 1.0, renorm: bool = True):
    """softmax -> top-k -> renormalise (-> scale): the router of BASELINE configs."""
    z = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, axis=1)
    if renorm:
        w = w / w.sum(axis=1, keepdims=True)
    return ids.astype(np.int64), (w * scale).astype(np.float32)


def zipf_topk(rng: np.random.Generator, tokens: int, experts: int, k: int, s: float = 1.2, tau: float = 1.0):
    """Skewed routing: expert popularity ~ rank^-s over a random permutation,
    per-token top-k by Gumbel-top-k on log p / tau (sampling without replacement)."""
    perm = rng.permutation(experts)
    p = np.empty(experts)
    p[perm] = np.arange(1, experts + 1, dtype=np.float64) ** (-s)
    p /= p.sum()
    logits = np.log(p)[None, :] / tau + rng.gumbel(size=(tokens, experts))
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    sel = np.take_along_axis(logits, ids, axis=1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    return ids.astype(np.int64), w.astype(np.float32)


def w8a8_case(seed: int, tokens: int, hidden: int, inter: int, experts: int, top_k: int, *, x_std: float = 1.0,
              int_range: int = 127, skew: float | None = None):
    """Random W8A8 layer: x bf16 bits, ids, weights, int8 weights + fp32 channel scales."""
    rng = np.random.default_rng(seed)
    x = bf16_bits(rng.standard_normal((tokens, hidden)).astype(np.float32) * x_std)
    if skew is None:
        ids, w = softmax_topk(rng.standard_normal((tokens, experts)).astype(np.float32), top_k)
    else:
        ids, w = zipf_topk(rng, tokens, experts, top_k, s=skew)
    q13 = rng.integers(-int_range, int_range + 1, size=(experts, 2 * inter, hidden), dtype=np.int8)
    q2 = rng.integers(-int_range, int_range + 1, size=(experts, hidden, inter), dtype=np.int8)
    # Channel scales near what per-channel quantisation of N(0, 0.02) weights gives.
    s13 = (rng.uniform(0.5, 1.5, size=(experts, 2 * inter)) * 0.08 / 127).astype(np.float32)
    s2 = (rng.uniform(0.5, 1.5, size=(experts, hidden)) * 0.08 / 127).astype(np.float32)
    return x, ids, w, q13, s13, q2, s2


# ------------------------------------------------------------ C-ABI runs --


def _t(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def pack_gpu(w: np.ndarray, n_groups: int, device):
    """Pack [E, N, K] int8 (or uint16 bf16 bits) weights through fcmoe_pack_experts."""
    import torch

    from fused_cpp_amd import cabi

    eb = 1 if w.dtype == np.int8 else 2
    e, n, k = w.shape
    src = _t(w.view(np.int16) if eb == 2 else w, device)
    per = cabi.lib().fcmoe_packed_expert_bytes(eb, n, k, n_groups)
    dst = torch.empty((e, per), dtype=torch.int8, device=device)
    cabi.check(cabi.lib().fcmoe_pack_experts(src.data_ptr(), eb, e, n, k, n_groups, dst.data_ptr(),
                                            cabi.stream_handle()), "pack")
    return dst


def gpu_route_build(ids: np.ndarray, experts: int, shared_id: int, device, ids_i64: bool = True):
    import torch

    from fused_cpp_amd import cabi

    L = cabi.lib()
    tokens, top_k = ids.shape
    kt = top_k + (1 if shared_id >= 0 else 0)
    ids_t = _t(ids.astype(np.int64 if ids_i64 else np.int32), device)
    counts = torch.empty(experts, dtype=torch.int32, device=device)
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=device)
    sorted_routes = torch.full((tokens * kt,), -1, dtype=torch.int32, device=device)
    # a stale value: the route build writes the count, it does not add to it
    invalid = torch.full((1,), 12345, dtype=torch.int32, device=device)
    wsb = L.fcmoe_route_workspace_bytes(tokens, top_k, experts, shared_id)
    ws = torch.empty(wsb, dtype=torch.uint8, device=device)
    cabi.check(L.fcmoe_route_build(ids_t.data_ptr(), 1 if ids_i64 else 0, tokens, top_k, experts, shared_id,
                                   counts.data_ptr(), offsets.data_ptr(), sorted_routes.data_ptr(),
                                   invalid.data_ptr(), ws.data_ptr(), wsb, cabi.stream_handle()), "route_build")
    torch.cuda.synchronize()
    return (counts.cpu().numpy(), offsets.cpu().numpy(), sorted_routes.cpu().numpy(), int(invalid.item()))


def gpu_quant_rows(x: np.ndarray, rounding: int, device, ldq: int | None = None):
    import torch

    from fused_cpp_amd import cabi

    rows, cols = x.shape
    ldq = ldq or cols
    is_f32 = 1 if x.dtype == np.float32 else 0
    xt = _t(x.view(np.int16) if x.dtype == np.uint16 else x, device)
    q = torch.full((rows, ldq), 99, dtype=torch.int8, device=device)
    s = torch.empty(rows, dtype=torch.float32, device=device)
    cabi.check(cabi.lib().fcmoe_quantize_rows(xt.data_ptr(), is_f32, rows, cols, rounding, q.data_ptr(), ldq,
                                              s.data_ptr(), cabi.stream_handle()), "quantize_rows")
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, device, *, shared_id: int = -1, scale: float = 1.0,
                     ids_i64: bool = True, packed=None, stages: bool = False, valid_experts: int | None = None,
                     noalloc: bool = False):
    """Run fcmoe_w8a8_forward (fcmoe_w8a8_forward_noalloc with noalloc=True);
    returns out bf16 bits (and stage buffers)."""
    import torch

    from fused_cpp_amd import cabi

    L = cabi.lib()
    tokens, hidden = x.shape
    experts, two_i, _ = q13.shape
    inter = two_i // 2
    if packed is None:
        packed = (pack_gpu(q13, 2, device), pack_gpu(q2, 1, device))
    p13, p2 = packed
    xt = _t(x.view(np.int16), device)
    idt = _t(ids.astype(np.int64 if ids_i64 else np.int32), device) if ids.shape[1] else None
    wt = _t(w.astype(np.float32), device) if ids.shape[1] else None
    s13t, s2t = _t(s13, device), _t(s2, device)
    out = torch.empty((tokens, hidden), dtype=torch.int16, device=device)
    inv = torch.zeros(1, dtype=torch.int32, device=device)
    a = cabi.MoeArgs()
    a.x = xt.data_ptr()
    a.tokens, a.hidden, a.inter = tokens, hidden, inter
    a.topk_ids = idt.data_ptr() if idt is not None else None
    a.ids_is_i64 = 1 if ids_i64 else 0
    a.topk_weights = wt.data_ptr() if wt is not None else None
    a.top_k = ids.shape[1]
    a.experts = experts
    a.valid_experts = valid_experts or experts
    a.shared_expert_id = shared_id
    a.routed_scaling = scale
    a.w13, a.w2 = p13.data_ptr(), p2.data_ptr()
    a.w13_scale, a.w2_scale = s13t.data_ptr(), s2t.data_ptr()
    a.activation = cabi.FCMOE_ACT_SILU_CLAMP10
    a.out = out.data_ptr()
    a.invalid_count = inv.data_ptr()
    if noalloc:
        if stages:
            raise ValueError("stage views need a caller workspace")
        cabi.check(L.fcmoe_w8a8_forward_noalloc(ctypes.byref(a), cabi.stream_handle()), "w8a8_forward_noalloc")
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.uint16)
    wsb = L.fcmoe_w8a8_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(wsb, dtype=torch.uint8, device=device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), wsb
    cabi.check(L.fcmoe_w8a8_forward(ctypes.byref(a), cabi.stream_handle()), "w8a8_forward")
    torch.cuda.synchronize()
    res = out.cpu().numpy().view(np.uint16)
    if not stages:
        return res
    views = [ctypes.c_void_p() for _ in range(7)]
    ldy, ldq = ctypes.c_int64(), ctypes.c_int64()
    cabi.check(L.fcmoe_w8a8_stage_views(ctypes.byref(a), ctypes.byref(views[0]), ctypes.byref(views[1]),
                                        ctypes.byref(ldy), ctypes.byref(views[2]), ctypes.byref(ldq),
                                        ctypes.byref(views[3]), ctypes.byref(views[4])), "stage_views")
    kt = ids.shape[1] + (1 if shared_id >= 0 else 0)
    R = tokens * kt

    def grab(p, n, dtype):
        t = torch.empty(n, dtype=dtype, device=device)
        cabi_copy(t, p.value, n * t.element_size())
        return t.cpu().numpy()

    st = {
        "sorted_routes": grab(views[0], R, torch.int32),
        "y": grab(views[1], R * ldy.value, torch.int16).view(np.uint16).reshape(R, ldy.value)[:, :inter],
        "q2": grab(views[2], R * ldq.value, torch.int8).reshape(R, ldq.value)[:, :inter],
        "s2row": grab(views[3], R, torch.float32),
        "route_out": grab(views[4], R * hidden, torch.float32).reshape(R, hidden),
        "invalid": int(inv.item()),
    }
    return res, st


def cabi_copy(dst, src_ptr: int, nbytes: int) -> None:
    """Device-to-device copy from a raw pointer into a torch tensor."""
    import torch

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    rc = hip.hipMemcpy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src_ptr), nbytes, 3)  # DeviceToDevice
    assert rc == 0, f"hipMemcpy failed: {rc}"


def gpu_grouped_gemm_acc(a: np.ndarray, row_map, counts: np.ndarray, w: np.ndarray, device):
    """Raw int32 accumulators of the grouped int8 GEMM for rows grouped by expert."""
    import torch

    from fused_cpp_amd import cabi

    L = cabi.lib()
    rows_a, k = a.shape
    lda = ((k + 63) // 64) * 64
    a_pad = np.zeros((rows_a, lda), np.int8)
    a_pad[:, :k] = a
    experts, n, _ = w.shape
    offsets = np.zeros(experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    total = int(offsets[-1])
    at = _t(a_pad, device)
    rm = _t(np.asarray(row_map, np.int32), device) if row_map is not None else None
    ct, ot = _t(counts.astype(np.int32), device), _t(offsets, device)
    pw = pack_gpu(w, 1, device)
    acc = torch.full((max(total, 1), n), -7, dtype=torch.int32, device=device)
    wsb = L.fcmoe_grouped_gemm_workspace_bytes(experts, total)
    ws = torch.empty(wsb, dtype=torch.uint8, device=device)
    cabi.check(L.fcmoe_grouped_gemm_i8_acc(at.data_ptr(), lda, rm.data_ptr() if rm is not None else None,
                                           ct.data_ptr(), ot.data_ptr(), experts, total, pw.data_ptr(), n, k,
                                           acc.data_ptr(), ws.data_ptr(), wsb, cabi.stream_handle()),
               "grouped_gemm_i8_acc")
    torch.cuda.synchronize()
    return acc.cpu().numpy()[:total], offsets


def gpu_bf16_forward(x, ids, w, w13, w2, device, *, shared_id: int = -1, scale: float = 1.0,
                     activation: int = 0, valid_experts: int | None = None):
    """Run fcmoe_bf16_forward through the C ABI on bf16-valued float32 inputs.
    Returns (out bf16 bits [T, H], route_pos [R], route_weight [R], route_out [R, H])."""
    import torch

    from fused_cpp_amd import cabi

    L = cabi.lib()
    tokens, hidden = x.shape
    experts, two_i, _ = w13.shape
    inter = two_i // 2
    p13 = pack_gpu(bf16_bits(w13).reshape(w13.shape), 2, device)
    p2 = pack_gpu(bf16_bits(w2).reshape(w2.shape), 1, device)
    xt = _t(bf16_bits(x).view(np.int16).reshape(x.shape), device)
    top_k = ids.shape[1]
    idt = _t(ids.astype(np.int64), device) if top_k else None
    wt = _t(w.astype(np.float32), device) if top_k else None
    out = torch.empty((tokens, hidden), dtype=torch.int16, device=device)
    a = cabi.MoeArgs()
    a.x = xt.data_ptr()
    a.tokens, a.hidden, a.inter = tokens, hidden, inter
    a.topk_ids = idt.data_ptr() if idt is not None else None
    a.ids_is_i64 = 1
    a.topk_weights = wt.data_ptr() if wt is not None else None
    a.top_k = top_k
    a.experts = experts
    a.valid_experts = valid_experts or experts
    a.shared_expert_id = shared_id
    a.routed_scaling = scale
    a.w13, a.w2 = p13.data_ptr(), p2.data_ptr()
    a.activation = activation
    a.out = out.data_ptr()
    wsb = L.fcmoe_bf16_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(wsb, dtype=torch.uint8, device=device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), wsb
    cabi.check(L.fcmoe_bf16_forward(ctypes.byref(a), cabi.stream_handle()), "bf16_forward")
    torch.cuda.synchronize()
    views = [ctypes.c_void_p() for _ in range(3)]
    cabi.check(L.fcmoe_bf16_stage_views(ctypes.byref(a), 0, ctypes.byref(views[0]), ctypes.byref(views[1]),
                                        ctypes.byref(views[2])), "bf16_stage_views")
    kt = top_k + (1 if shared_id >= 0 else 0)
    R = tokens * kt

    def grab(p, n, dtype):
        t = torch.empty(n, dtype=dtype, device=device)
        cabi_copy(t, p.value, n * t.element_size())
        return t.cpu().numpy()

    return (out.cpu().numpy().view(np.uint16), grab(views[0], R, torch.int32), grab(views[1], R, torch.float32),
            grab(views[2], R * hidden, torch.float32).reshape(R, hidden))


def w8a8_layer_staged(x_bits, ids, topk_w, experts: int, shared_id: int, routed_scale: float, gemm13, gemm2,
                      s13_of, s2_of):
    """The oracle's W8A8 layer (orc_w8a8_forward) with its two GEMMs supplied
    by the caller: every other step (token quantisation, W13 epilogue and
    requant, store_w2, ordered merge) is the oracle's own C code. gemm13(e,
    a [rows, H] int8) and gemm2(e, q2 [rows, I] int8) must return the exact
    int32 accumulators [rows, N] of expert e (any exact integer GEMM gives
    the same values); s13_of(e) / s2_of(e) return its channel scales. Routes
    with ids outside [0, experts) contribute nothing, as in the oracle."""
    import oracle

    T, k = ids.shape
    shared = shared_id >= 0
    kt = k + (1 if shared else 0)
    xq, xs = oracle.quant_rows_away(x_bits)
    route_expert = np.concatenate([ids, np.full((T, 1), shared_id)], 1) if shared else ids
    route_expert = route_expert.reshape(-1)
    hidden = x_bits.shape[1]
    route_out = np.zeros((T * kt, hidden), np.float32)
    valid = (route_expert >= 0) & (route_expert < experts)
    order = np.argsort(np.where(valid, route_expert, experts), kind="stable")
    bounds = np.searchsorted(route_expert[order], np.arange(experts + 1)) if valid.any() else None
    for e in range(experts):
        if bounds is None:
            break
        r = order[bounds[e]:bounds[e + 1]]
        r = r[route_expert[r] == e]
        if r.size == 0:
            continue
        tok = r // kt
        acc13 = gemm13(e, xq[tok])
        q2, s2row = oracle.w8a8_w13_rows(acc13, xs[tok], s13_of(e))
        acc2 = gemm2(e, q2)
        route_out[r] = oracle.w8a8_w2_rows(acc2, s2row, s2_of(e))
    rw = oracle.w8a8_route_weights(topk_w, shared, routed_scale)
    return oracle.w8a8_merge(route_out, rw, T, kt)
