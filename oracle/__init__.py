"""CPU oracle for the fused-MoE hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the checker (or the timed CPU baseline).
The product package ``fused_cpp_amd`` never imports it.

Two parts:

* ``liboracle.so`` (built from ``fcmoe_oracle.c`` by ``make -C oracle``): the
  W8A8 pipeline, routing, activation/weight quantisation and i8gemm, restated
  from the reference one binary32 operation at a time (see the citations in the
  C file). Wrapped here with ctypes + numpy.
* ``router_topk``: numpy restatement of the caller-side router (softmax ->
  top-k -> renormalise -> scale) that produces the MoE op's ids and weights.
* ``bf16_moe_reference``: an fp32 numpy restatement of the BF16 fused MoE
  semantics of ``src/fused_cpp/moe/naive.py:161-272`` (grouped per-expert
  linear, activation, weighted top-k sum) used as the tolerance reference.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile."""
    cmd = ["make", "-C", str(_HERE)] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(_LIB_PATH))
        l.orc_fexpa_exp_neg.restype = _F
        l.orc_fexpa_exp_neg.argtypes = [_F]
        l.orc_fexpa_entry.restype = ctypes.c_uint32
        l.orc_fexpa_entry.argtypes = [_I]
        l.orc_f32_to_bf16.restype = ctypes.c_uint16
        l.orc_f32_to_bf16.argtypes = [_F]
        l.orc_quant_row_away.argtypes = [_P, _I, _P, _P]
        l.orc_quant_row_even.argtypes = [_P, _I, _I, _P, _P]
        l.orc_quant_weight_rows.argtypes = [_P, _I64, _I, _P, _P]
        l.orc_route_build.restype = _I64
        l.orc_route_build.argtypes = [_P, _I64, _I64, _I64, _I64, _P, _P, _P]
        l.orc_w8a8_forward.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _F, _P,
                                       _P, _P, _P, _P, _P, _P]
        l.orc_w8a8_expert_range.restype = _I64
        l.orc_w8a8_expert_range.argtypes = [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _P]
        l.orc_w8a8_w13_rows.argtypes = [_P, _I64, _I64, _P, _P, _P, _P, _P]
        l.orc_w8a8_w2_rows.argtypes = [_P, _I64, _I64, _P, _P, _P]
        l.orc_w8a8_merge.argtypes = [_P, _P, _I64, _I64, _I64, _P]
        l.orc_gemm_i8_rows.argtypes = [_P, _I64, _P, _I64, _P, _I64, _I64, _P]
        l.orc_i8gemm.argtypes = [_P, _I, _I64, _I64, _P, _P, _I64, _P, _I, _P]
        l.orc_bf16_activation.argtypes = [_P, _I64, _I64, _I, _P]
        l.orc_bf16_route_merge.argtypes = [_P, _P, _I64, _I64, _I64, _P]
        _lib = l
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- bf16 <-> fp32 helpers (numpy, uint16 bit patterns) -------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even by integer bias (kernels.cpp:194-198)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> 16) & 1
    return ((u + np.uint32(0x7FFF) + lsb) >> 16).astype(np.uint16)


# ---- scalar / row primitives ------------------------------------------------

def fexpa_exp_neg(g: float) -> float:
    return float(lib().orc_fexpa_exp_neg(float(g)))


def fexpa_table() -> np.ndarray:
    return np.array([lib().orc_fexpa_entry(i) for i in range(64)], dtype=np.uint32)


def quant_rows_away(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantize_bf16_row per row (half away from zero, x * (1/scale))."""
    x_bits = _c(x_bits, np.uint16)
    rows, n = x_bits.shape
    q = np.empty((rows, n), np.int8)
    s = np.empty(rows, np.float32)
    L = lib()
    for r in range(rows):
        L.orc_quant_row_away(_ptr(x_bits[r]), n, _ptr(q[r]), s[r:].ctypes.data_as(ctypes.c_void_p))
    return q, s


def quant_rows_even(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """i8gemm per-row quantisation (ties to even, x / scale). x: uint16 bf16 bits or float32."""
    is_f32 = 1 if x.dtype == np.float32 else 0
    x = _c(x, np.float32 if is_f32 else np.uint16)
    rows, n = x.shape
    q = np.empty((rows, n), np.int8)
    s = np.empty(rows, np.float32)
    L = lib()
    for r in range(rows):
        L.orc_quant_row_even(_ptr(x[r]), is_f32, n, _ptr(q[r]), s[r:].ctypes.data_as(ctypes.c_void_p))
    return q, s


def quant_weight_rows(w_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric int8 (kernels.cpp:451-457). w_bits: [..., K] bf16 bits."""
    w_bits = _c(w_bits, np.uint16)
    shape = w_bits.shape
    rows = int(np.prod(shape[:-1]))
    q = np.empty(shape, np.int8)
    s = np.empty(shape[:-1], np.float32)
    lib().orc_quant_weight_rows(_ptr(w_bits), rows, shape[-1], _ptr(q), _ptr(s))
    return q, s


def router_topk(logits: np.ndarray, k: int, *, renormalize: bool = True, scale: float = 1.0):
    """Caller-side router (docs/vllm_bf16_tiled_moe_integration.md:75-87; the reference
    itself receives ids/weights, src/fused_cpp/moe/bf16_tiled.py:676-681), in fp32:
    p = exp(x - max) / sum(exp(x - max)); ids = the k largest logits in descending order,
    the lower expert id first on ties; w = p[ids] (/ sum p[ids]) * scale."""
    x = np.asarray(logits, np.float32)
    z = np.exp(x - x.max(axis=1, keepdims=True))
    p = z / z.sum(axis=1, keepdims=True, dtype=np.float32)
    ids = np.argsort(-x, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, axis=1)
    if renormalize:
        w = w / w.sum(axis=1, keepdims=True, dtype=np.float32)
    return ids.astype(np.int64), (w * np.float32(scale)).astype(np.float32)


def route_build(ids: np.ndarray, experts: int, shared_id: int = -1):
    """Per-expert ascending flat-route lists. Returns (counts, offsets, sorted_routes, n_invalid)."""
    ids = _c(ids, np.int64)
    tokens, top_k = ids.shape
    kt = top_k + (1 if shared_id >= 0 else 0)
    counts = np.empty(experts, np.int64)
    offsets = np.empty(experts + 1, np.int64)
    sorted_routes = np.full(tokens * kt, -1, np.int64)
    bad = lib().orc_route_build(_ptr(ids), tokens, top_k, experts, shared_id, _ptr(counts), _ptr(offsets),
                                _ptr(sorted_routes))
    return counts, offsets, sorted_routes[: int(offsets[-1])], int(bad)


def gemm_i8_rows(a: np.ndarray, rows: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact int32 acc[j, n] = sum_k a[rows[j], k] * w[n, k]."""
    a = _c(a, np.int8)
    w = _c(w, np.int8)
    rows = _c(rows, np.int64)
    n, k = w.shape
    acc = np.empty((rows.size, n), np.int32)
    lib().orc_gemm_i8_rows(_ptr(a), a.shape[1], _ptr(rows), rows.size, _ptr(w), n, k, _ptr(acc))
    return acc


def w8a8_forward(x_bits, ids, topk_w, w13, s13, w2, s2, *, shared_id: int = -1, routed_scale: float = 1.0,
                 dumps: bool = False):
    """Full W8A8 fused MoE forward (kernels.cpp:463-694). Returns out bits [T,H] (and a dict of stage dumps)."""
    x_bits = _c(x_bits, np.uint16)
    ids = _c(ids, np.int64)
    topk_w = _c(topk_w, np.float32)
    w13 = _c(w13, np.int8)
    w2 = _c(w2, np.int8)
    s13 = _c(s13, np.float32)
    s2 = _c(s2, np.float32)
    tokens, hidden = x_bits.shape
    top_k = ids.shape[1]
    experts, two_i, _ = w13.shape
    inter = two_i // 2
    kt = top_k + (1 if shared_id >= 0 else 0)
    routes = tokens * kt
    out = np.empty((tokens, hidden), np.uint16)
    d = {}
    if dumps:
        d = {
            "acc13": np.zeros((routes, 2 * inter), np.int32),
            "y": np.zeros((routes, inter), np.uint16),
            "q2": np.zeros((routes, inter), np.int8),
            "s2row": np.zeros(routes, np.float32),
            "acc2": np.zeros((routes, hidden), np.int32),
            "route_out": np.zeros((routes, hidden), np.float32),
        }
    lib().orc_w8a8_forward(
        _ptr(x_bits), _ptr(ids), _ptr(topk_w), tokens, top_k, hidden, inter, experts, _ptr(w13), _ptr(s13),
        _ptr(w2), _ptr(s2), shared_id, routed_scale, _ptr(out), _ptr(d.get("acc13")), _ptr(d.get("y")),
        _ptr(d.get("q2")), _ptr(d.get("s2row")), _ptr(d.get("acc2")), _ptr(d.get("route_out")))
    return (out, d) if dumps else out


def w8a8_w13_rows(acc13, xs, s13e, want_y: bool = False):
    """The W8A8 stages after W13 for rows of one expert (kernels.cpp:230-246,
    211-228): acc13 [rows, 2I] int32, xs [rows] token scales, s13e [2I] ->
    (q2 [rows, I] int8, s2row [rows] fp32[, y bf16 bits])."""
    acc13 = _c(acc13, np.int32)
    rows, two_i = acc13.shape
    inter = two_i // 2
    q2 = np.empty((rows, inter), np.int8)
    s2row = np.empty(rows, np.float32)
    y = np.empty((rows, inter), np.uint16) if want_y else None
    lib().orc_w8a8_w13_rows(_ptr(acc13), rows, inter, _ptr(_c(xs, np.float32)), _ptr(_c(s13e, np.float32)), _ptr(y),
                            _ptr(q2), _ptr(s2row))
    return (q2, s2row, y) if want_y else (q2, s2row)


def w8a8_w2_rows(acc2, s2row, s2e, out=None):
    """store_w2 (kernels.cpp:248-257) for rows of one expert: acc2 [rows, H] int32 -> fp32 route rows."""
    acc2 = _c(acc2, np.int32)
    rows, hidden = acc2.shape
    if out is None:
        out = np.empty((rows, hidden), np.float32)
    assert out.dtype == np.float32 and out.flags.c_contiguous and out.shape == (rows, hidden)
    lib().orc_w8a8_w2_rows(_ptr(acc2), rows, hidden, _ptr(_c(s2row, np.float32)), _ptr(_c(s2e, np.float32)),
                           _ptr(out))
    return out


def w8a8_route_weights(topk_w, shared: bool, routed_scale: float) -> np.ndarray:
    """Per flat route merge weights as orc_w8a8_forward forms them (bf16_tiled.py:1007-1013):
    routed weights x routed_scale with a shared slot of weight 1, else the weights as given."""
    topk_w = _c(topk_w, np.float32)
    if not shared:
        return topk_w.reshape(-1).copy()
    t, k = topk_w.shape
    rw = np.ones((t, k + 1), np.float32)
    rw[:, :k] = topk_w * np.float32(routed_scale)
    return rw.reshape(-1)


def w8a8_merge(route_out, rw, tokens: int, kt: int) -> np.ndarray:
    """Ordered-FMA merge (kernels.cpp:674-688): route_out [T*kt, H] fp32 by flat route -> bf16 bits [T, H]."""
    route_out = _c(route_out, np.float32)
    hidden = route_out.shape[1]
    out = np.empty((tokens, hidden), np.uint16)
    lib().orc_w8a8_merge(_ptr(route_out), _ptr(_c(rw, np.float32)), tokens, kt, hidden, _ptr(out))
    return out


def w8a8_expert_range(x_bits, sorted_routes, offsets, kt, w13, s13, w2, s2, e_begin, e_end, route_out):
    """Grouped per-expert W8A8 work for experts [e_begin, e_end); fills route_out rows. Returns rows done."""
    experts, two_i, hidden = w13.shape
    return int(lib().orc_w8a8_expert_range(
        _ptr(x_bits), _ptr(sorted_routes), _ptr(offsets), kt, hidden, two_i // 2, _ptr(w13), _ptr(s13), _ptr(w2),
        _ptr(s2), e_begin, e_end, _ptr(route_out)))


def i8gemm(x: np.ndarray, w: np.ndarray, w_scale: np.ndarray, bias: np.ndarray | None, out_bf16: bool):
    """i8gemm.dynamic_scaled_mm generic semantics. x: [M,K] float32 or uint16 bf16 bits; w [N,K] int8."""
    is_f32 = 1 if x.dtype == np.float32 else 0
    x = _c(x, np.float32 if is_f32 else np.uint16)
    w = _c(w, np.int8)
    m, k = x.shape
    n = w.shape[0]
    ws = _c(np.broadcast_to(np.asarray(w_scale, np.float32).reshape(-1), (n,)), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    out = np.empty((m, n), np.uint16 if out_bf16 else np.float32)
    lib().orc_i8gemm(_ptr(x), is_f32, m, k, _ptr(w), _ptr(ws), n, _ptr(b), 1 if out_bf16 else 0, _ptr(out))
    return out


_ACT_MODES = {"silu": 0, "gelu": 1, "swigluoai": 2, "silu_clamp10": 3}


def bf16_activation(gate_up: np.ndarray, mode: str) -> np.ndarray:
    gate_up = _c(gate_up, np.float32)
    rows, two_f = gate_up.shape
    y = np.empty((rows, two_f // 2), np.uint16)
    lib().orc_bf16_activation(_ptr(gate_up), rows, two_f // 2, _ACT_MODES[mode], _ptr(y))
    return y


def bf16_route_merge(route_out: np.ndarray, weights: np.ndarray, kt: int) -> np.ndarray:
    """BF16 executor's top-k merge (csrc/moe/arm/sve_bf16/route_merge.cpp:38-126):
    route_out [T*kt, H] fp32 rows by flat route, weights [T*kt] fp32 -> bf16
    bits [T, H]. kt in {2,4,6,8}: weighted leaves summed as a power-of-two
    split tree; otherwise an ordered fused multiply-add chain."""
    route_out = _c(route_out, np.float32)
    weights = _c(weights, np.float32).reshape(-1)
    rows, hidden = route_out.shape
    tokens = rows // kt
    out = np.empty((tokens, hidden), np.uint16)
    lib().orc_bf16_route_merge(_ptr(route_out), _ptr(weights), tokens, kt, hidden, _ptr(out))
    return out


# ---- BF16 fused MoE fp32 reference -----------------------------------------

def _act_f32(gate_up: np.ndarray, mode: str) -> np.ndarray:
    f = gate_up.shape[-1] // 2
    if mode == "swigluoai":
        gate = np.minimum(gate_up[:, ::2], 7.0)
        up = np.clip(gate_up[:, 1::2], -7.0, 7.0)
        return (up + 1.0) * (gate / (1.0 + np.exp(-gate * 1.702)))
    gate, up = gate_up[:, :f], gate_up[:, f:]
    if mode == "silu_clamp10":
        gate = np.minimum(gate, 10.0)
        up = np.clip(up, -10.0, 10.0)
    if mode == "gelu":
        from scipy.special import erf

        return 0.5 * gate * (1.0 + erf(gate / np.sqrt(2.0))) * up
    return gate / (1.0 + np.exp(-gate)) * up


def bf16_moe_reference(x: np.ndarray, w13: np.ndarray, w2: np.ndarray, topk_w: np.ndarray, ids: np.ndarray, *,
                       w13_bias=None, w2_bias=None, activation: str = "silu", skip_weighted: bool = False,
                       round_intermediate: bool = False) -> np.ndarray:
    """fp32 restatement of fused_moe_naive (src/fused_cpp/moe/naive.py:161-272).

    x [T,H], w13 [E,2F,H], w2 [E,H,F] as float32 arrays (already bf16-valued);
    returns float32 [T,H] before the final bf16 cast. ``round_intermediate``
    rounds the activation output to bf16 as the native executors do
    (fused_moe_bf16_tiled.cpp:1861-1874).
    """
    x = np.asarray(x, np.float32)
    tokens, hidden = x.shape
    top_k = ids.shape[1]
    out_routes = np.zeros((tokens, top_k, hidden), np.float32)
    flat = ids.reshape(-1).astype(np.int64)
    for e in np.unique(flat):
        sel = np.nonzero(flat == e)[0]
        rows = x[sel // top_k]
        gu = rows @ w13[e].astype(np.float32).T
        if w13_bias is not None:
            gu = gu + w13_bias[e].astype(np.float32)
        y = _act_f32(gu.astype(np.float32), activation).astype(np.float32)
        if round_intermediate:
            y = bf16_bits_to_f32(f32_to_bf16_bits(y))
        o = y @ w2[e].astype(np.float32).T
        if w2_bias is not None:
            o = o + w2_bias[e].astype(np.float32)
        out_routes[sel // top_k, sel % top_k] = o
    if skip_weighted:
        return out_routes[:, 0, :]
    return (out_routes * topk_w.astype(np.float32)[:, :, None]).sum(axis=1)
