"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for the fused quantized MoE layer.

A restatement of the reference algorithms in numpy (byte/integer/fp32 element
arithmetic, whole tensors) and in C (``oracle_core.c``: per-element dequant,
the router dot products in the GPU's fixed summation order, and the expert
SwiGLU in double precision).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker; the product (``freetoken-intel_amd/ftmoe``) never does.

Pins (see tests/test_oracle.py): the reference's known-answer tests
(tests/test_gptq_quant.py:31-69, tests/test_mxfp4_quant.py:23-46,
tests/test_weight_gptq_banks.py:90-111), the OCP e4m3 definition checked
against torch.float8_e4m3fn for all 256 codes, exact integer/power-of-two
closed forms, brute-force float64 loops on tiny inputs, and the reference's
own CPU MoE kernel (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp, built
unmodified into oracle/_ref) for the SwiGLU + weighted combine.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libcpu_moe_ref.so")

F_BF16, F_FP8, F_GPTQ, F_INT8, F_MXFP4, F_FP32 = 0, 1, 2, 3, 4, 5
D_F32, D_F16, D_BF16 = 0, 1, 2
ACTS = {"silu": 0, "swiglu": 0, "swish": 0, "gelu": 1, "relu": 2, "swiglu_oai": 3}
FMT_CODES = {"bf16": F_BF16, "fp8_block": F_FP8, "gptq_int4": F_GPTQ, "int8_channel": F_INT8, "mxfp4": F_MXFP4,
             "fp32": F_FP32}


class OrcProj(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("z", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("w_stride", ctypes.c_int64), ("s_stride", ctypes.c_int64), ("z_stride", ctypes.c_int64),
        ("bias_stride", ctypes.c_int64), ("fmt", ctypes.c_int32), ("s_dtype", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32), ("group", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
        ("num_slots", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-C", HERE, "liboracle.so"], check=True, capture_output=True)
        L = ctypes.CDLL(LIB_PATH)
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        L.orc_deq.restype = ctypes.c_float
        L.orc_deq.argtypes = [ctypes.POINTER(OrcProj), i32, i32, i32]
        L.orc_dequant.restype = None
        L.orc_dequant.argtypes = [ctypes.POINTER(OrcProj), i32, vp]
        L.orc_router_logits.restype = None
        L.orc_router_logits.argtypes = [vp, i32, i32, vp, i32, vp, vp]
        L.orc_expert_forward.restype = ctypes.c_int
        L.orc_expert_forward.argtypes = [ctypes.POINTER(OrcProj), ctypes.POINTER(OrcProj), i32, vp, i32, i32,
                                         ctypes.c_float, ctypes.c_float, i32, vp]
        L.orc_moe_experts.restype = ctypes.c_int
        L.orc_moe_experts.argtypes = [ctypes.POINTER(OrcProj), ctypes.POINTER(OrcProj), vp, i32, vp, i32, i32, vp, vp,
                                      i32, ctypes.c_float, ctypes.c_float, i32, i32, i32, vp]
        L.orc_e4m3_to_f32.restype = ctypes.c_float
        L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_e8m0_to_f32.restype = ctypes.c_float
        L.orc_e8m0_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_act.restype = ctypes.c_double
        L.orc_act.argtypes = [i32, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double]
        L.orc_expf.restype = ctypes.c_float
        L.orc_expf.argtypes = [ctypes.c_float]
        L.orc_expf_n.restype = None
        L.orc_expf_n.argtypes = [vp, ctypes.c_int64, vp]
        L.orc_sigmoidf.restype = ctypes.c_float
        L.orc_sigmoidf.argtypes = [ctypes.c_float]
        L.orc_round_f16.restype = ctypes.c_float
        L.orc_round_f16.argtypes = [ctypes.c_float]
        L.orc_wave_sum.restype = ctypes.c_float
        L.orc_wave_sum.argtypes = [vp]
        L.orc_route.restype = ctypes.c_int
        L.orc_route.argtypes = [vp, i32, i32, i32, i32, i32, i32, i32, vp, vp]
        _lib = L
    return _lib


# ----------------------------------------------------------------- bf16 / fp16
def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16), NaN -> quiet NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def round_to(a, dt: str) -> np.ndarray:
    if dt == "bf16":
        return round_bf16(a)
    if dt == "f16":
        return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(a, np.float32)


# ----------------------------------------------------------------- codes
def e4m3_lut() -> np.ndarray:
    """OCP FP8 e4m3fn value of each of the 256 codes (bias 7, subnormal m*2^-9, S.1111.111 = NaN)."""
    b = np.arange(256)
    s, e, m = b >> 7, (b >> 3) & 0xF, b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e.astype(np.float64) - 10))
    v = np.where(s == 1, -v, v)
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return v.astype(np.float32)


E4M3 = e4m3_lut()
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                dtype=np.float32)  # python/freetoken/kernel/triton/mxfp4_linear.py:38-41


def e8m0_to_f32(s) -> np.ndarray:
    """torch.exp2(s - 127) for e8m0 bytes (mxfp4_linear.py:74): 255 -> +inf, 0 -> 2^-127."""
    s = np.asarray(s).astype(np.int64)
    with np.errstate(over="ignore"):
        return np.ldexp(np.float32(1.0), s - 127).astype(np.float32)


def f32_to_e4m3(a) -> np.ndarray:
    """fp32 -> e4m3fn code, round-to-nearest-even; |a| above the 448 saturation
    midpoint and NaN give the NaN code, like torch's fp32 -> float8_e4m3fn cast."""
    a = np.asarray(a, dtype=np.float32)
    mag = np.abs(a).astype(np.float64)
    pos = E4M3[:127].astype(np.float64)  # codes 0x00..0x7E ascending
    idx = np.searchsorted(pos, mag)       # pos[idx-1] < mag <= pos[idx]
    hi = np.clip(idx, 0, 126)
    lo = np.clip(idx - 1, 0, 126)
    dlo, dhi = mag - pos[lo], pos[hi] - mag
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(mag == pos[lo], lo, code)
    over = mag > 464.0  # midpoint between 448 and the (absent) next value 480
    code = np.where(over | np.isnan(a), 0x7F, code)
    sign = np.signbit(a)
    return (code | np.where(sign, 0x80, 0)).astype(np.uint8)


# ----------------------------------------------------------------- dequant (numpy, whole tensors)
def dequantize_block_fp8(w_u8: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """python/freetoken/kernel/triton/fp8_block_linear.py:48-91 -> fp32 [N, K]."""
    N, K = w_u8.shape
    s = np.asarray(scale, np.float32)
    rows = np.arange(N) // block
    cols = np.arange(K) // block
    return E4M3[w_u8] * s[rows][:, cols]


def dequantize_gptq_int4(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group: int) -> np.ndarray:
    """python/freetoken/kernel/triton/gptq_linear.py:55-124 (desc_act=False) -> fp32 [K, N]."""
    qw = qweight.astype(np.int64) & 0xFFFFFFFF
    Kp, N = qw.shape
    K = Kp * 8
    shifts = (np.arange(8) * 4).reshape(1, 8, 1)
    q = ((qw[:, None, :] >> shifts) & 0xF).reshape(K, N)
    qz = qzeros.astype(np.int64) & 0xFFFFFFFF
    G = qz.shape[0]
    z = ((qz[:, :, None] >> (np.arange(8) * 4).reshape(1, 1, 8)) & 0xF).reshape(G, N) + 1
    g = np.arange(K) // group
    s = np.asarray(scales, np.float32)
    return s[g] * (q.astype(np.float32) - z[g].astype(np.float32))


def dequantize_int8_packed(weight_packed: np.ndarray, weight_scale: np.ndarray, k: int) -> np.ndarray:
    """python/freetoken/kernel/triton/int8_packed_linear.py:74-125 -> fp32 [N, K]."""
    wp = weight_packed.astype(np.int64) & 0xFFFFFFFF
    N, C = wp.shape
    b = ((wp[:, :, None] >> (np.arange(4) * 8).reshape(1, 1, 4)) & 0xFF).reshape(N, C * 4)[:, :k]
    v = (b - 128).astype(np.float32)
    ng = weight_scale.shape[1]
    g = np.arange(k) // (k // ng)
    return v * np.asarray(weight_scale, np.float32)[:, g]


def dequantize_mxfp4_blocks(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """python/freetoken/kernel/triton/mxfp4_linear.py:46-76 -> fp32 [..., K]."""
    nib = np.stack((blocks & 0x0F, blocks >> 4), axis=-1).reshape(*blocks.shape[:-1], 32)
    v = E2M1[nib] * e8m0_to_f32(scales)[..., None]
    return v.reshape(*blocks.shape[:-2], blocks.shape[-2] * 32).astype(np.float32)


# ----------------------------------------------------------------- quantizers (numpy)
def quantize_block_fp8(w: np.ndarray, block: int = 128):
    """fp8_block_linear.py:94-125 -> (e4m3 codes uint8 [N, K], fp32 scale)."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    nbr, nbc = -(-N // block), -(-K // block)
    p = np.zeros((nbr * block, nbc * block), np.float32)
    p[:N, :K] = w
    b = p.reshape(nbr, block, nbc, block)
    amax = np.maximum(np.abs(b).max(axis=(1, 3)), np.float32(1e-12))
    scale = (amax / np.float32(448.0)).astype(np.float32)
    q = np.clip(b / scale[:, None, :, None], -448.0, 448.0).astype(np.float32)
    return f32_to_e4m3(q.reshape(nbr * block, nbc * block)[:N, :K]), scale


def quantize_mxfp4_blocks(w: np.ndarray):
    """mxfp4_linear.py:79-111 -> (uint8 blocks [..., K/32, 16], uint8 e8m0 [..., K/32])."""
    w = np.asarray(w, np.float32)
    K = w.shape[-1]
    bf = w.reshape(*w.shape[:-1], K // 32, 32)
    amax = np.maximum(np.abs(bf).max(axis=-1), np.float32(1e-12))
    e = np.ceil(np.log2(amax / np.float32(6.0)))
    eb = np.clip(np.round(e + 127), 0, 254).astype(np.uint8)
    scaled = bf / e8m0_to_f32(eb)[..., None]
    nib = np.abs(scaled[..., None] - E2M1).argmin(axis=-1).astype(np.uint8)
    return (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8), eb


def quantize_int8_channel(w: np.ndarray):
    """int8_linear.py:34-43 -> (int8 codes, fp32 per-row scale)."""
    w = np.asarray(w, np.float32)
    amax = np.maximum(np.abs(w).max(axis=-1, keepdims=True), np.float32(1e-12))
    scale = (amax / np.float32(127)).astype(np.float32)
    q = np.clip(np.round(w / scale), -127, 127).astype(np.int8)
    return q, scale[..., 0]


def pack_int8(codes: np.ndarray) -> np.ndarray:
    """Offset-binary int8 pack, 4 per int32 (inverse of int8_packed_linear.py:74-93)."""
    b = (codes.astype(np.int64) + 128).reshape(*codes.shape[:-1], codes.shape[-1] // 4, 4)
    word = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)
    return word.astype(np.uint32).view(np.int32)


# ----------------------------------------------------------------- routing (numpy)
def _select(key: np.ndarray, k: int) -> np.ndarray:
    """Top-k indices per row, ordered by (key desc, index asc)."""
    T, E = key.shape
    out = np.empty((T, k), np.int64)
    idx = np.arange(E)
    for t in range(T):
        order = np.lexsort((idx, -key[t].astype(np.float64)))
        out[t] = order[:k]
    return out


_ROUTE_MODES = {"softmax_topk": 0, "softmax_topk_lowp": 1, "topk_softmax": 2}
_DT = {"f32": D_F32, "fp32": D_F32, "f16": D_F16, "bf16": D_BF16}


def route(logits: np.ndarray, k: int, mode: str = "softmax_topk", renormalize: bool = True,
          weight_dt: str = "bf16", prob_dt: str = "bf16"):
    """Router softmax / top-k / renorm on fp32 logits (already rounded to the
    logits dtype), with the GPU kernel's IEEE operations step for step
    (``orc_route`` in oracle_core.c: its own e^x, the lane-order sums), so
    routing indices and router weights are bitwise comparable.

    * ``softmax_topk``      qwen3_5_moe/__init__.py:1225-1227 (fp32 softmax over E)
    * ``softmax_topk_lowp`` fused_moe.py:92-97, qwen3_moe/__init__.py:473-475 (softmax in the logits dtype)
    * ``topk_softmax``      gpt_oss/__init__.py:350-352 (top-k on logits, softmax over the k)
    Ties break to the lower expert index.  Returns (ids int32 [T,k], weights fp32 [T,k])."""
    l = np.ascontiguousarray(logits, np.float32)
    T, E = l.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    rc = lib().orc_route(l.ctypes.data, T, E, k, _ROUTE_MODES[mode], 1 if renormalize else 0, _DT[prob_dt],
                         _DT[weight_dt], ids.ctypes.data, w.ctypes.data)
    if rc != 0:
        raise ValueError(f"orc_route rc={rc} (T={T}, E={E}, k={k})")
    return ids, w


def route_f64(logits: np.ndarray, k: int, mode: str = "softmax_topk", renormalize: bool = True,
              weight_dt: str = "bf16", prob_dt: str = "bf16"):
    """The same routing with float64 exp and numpy sums: the textbook
    arithmetic :func:`route` is checked against (tests/test_oracle.py)."""
    l = np.asarray(logits, np.float32)
    if mode == "topk_softmax":
        ids = _select(l, k)
        v = np.take_along_axis(l, ids, axis=1).astype(np.float64)
        e = np.exp(v - v[:, :1])
        w = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
        return ids.astype(np.int32), round_to(w, weight_dt)
    m = l.max(axis=1, keepdims=True)
    e = np.exp((l - m).astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    if mode == "softmax_topk":
        ids = _select(l, k)
        w = np.take_along_axis(p, ids, axis=1)
        if renormalize:
            w = w / w.sum(axis=1, keepdims=True)
        return ids.astype(np.int32), round_to(w, weight_dt)
    pl = round_to(p, prob_dt)
    ids = _select(pl, k)
    w = np.take_along_axis(pl, ids, axis=1)
    if renormalize:
        w = round_to(w / round_to(w.sum(axis=1, keepdims=True), prob_dt), prob_dt)
    return ids.astype(np.int32), round_to(w, weight_dt)


def expf(x) -> np.ndarray:
    """The routing e^x (orc_expf) elementwise, fp32."""
    a = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(a)
    lib().orc_expf_n(a.ctypes.data, a.size, y.ctypes.data)
    return y


def sigmoidf(z) -> np.ndarray:
    """The shared expert's gate weight 1 / (1 + e^-z) on orc_expf, fp32."""
    f = lib().orc_sigmoidf
    a = np.asarray(z, np.float32)
    return np.array([f(float(v)) for v in a.ravel()], np.float32).reshape(a.shape)


def wave_sum(v64) -> float:
    """The kernel's 64-lane sum order (orc_wave_sum)."""
    a = np.ascontiguousarray(v64, np.float32)
    assert a.shape == (64,)
    return float(lib().orc_wave_sum(a.ctypes.data))


# ----------------------------------------------------------------- C-backed pieces
def act(name: str, g, u, alpha: float = 1.702, limit: float = 7.0) -> np.ndarray:
    """The expert activation h = act(g, u) of the C oracle (oracle_core.c act_d)
    in double precision, elementwise (fused_moe.py:53-61, gpt_oss/__init__.py:306-310)."""
    g = np.asarray(g, np.float64)
    u = np.broadcast_to(np.asarray(u, np.float64), g.shape)
    f, code = lib().orc_act, ACTS[name]
    return np.array([f(code, float(a), float(b), float(alpha), float(limit)) for a, b in zip(g.ravel(), u.ravel())],
                    np.float64).reshape(g.shape)



def _dt_code(arr: np.ndarray) -> int:
    if arr.dtype == np.float32:
        return D_F32
    if arr.dtype == np.float16:
        return D_F16
    return D_BF16  # uint16 bf16 bit patterns


@dataclass
class OracleProj:
    """numpy arrays of one projection bank (slot-stacked) + its C descriptor."""

    fmt: str
    w: np.ndarray
    N: int
    K: int
    s: Optional[np.ndarray] = None
    z: Optional[np.ndarray] = None
    bias: Optional[np.ndarray] = None  # bf16 bits uint16 [S, N] or float32
    group: int = 0

    def c(self) -> OrcProj:
        for name in ("w", "s", "z", "bias"):
            a = getattr(self, name)
            if a is not None and not a.flags["C_CONTIGUOUS"]:
                setattr(self, name, np.ascontiguousarray(a))
        p = OrcProj()
        p.w = self.w.ctypes.data
        p.s = self.s.ctypes.data if self.s is not None else None
        p.z = self.z.ctypes.data if self.z is not None else None
        p.bias = self.bias.ctypes.data if self.bias is not None else None
        slotted = self.w.ndim == (4 if self.fmt == "mxfp4" else 3)
        p.w_stride = self.w.strides[0] if slotted else 0
        p.s_stride = self.s.strides[0] if slotted and self.s is not None else 0
        p.z_stride = self.z.strides[0] if slotted and self.z is not None else 0
        p.bias_stride = self.bias.strides[0] if slotted and self.bias is not None else 0
        p.fmt = FMT_CODES[self.fmt]
        p.s_dtype = _dt_code(self.s) if self.s is not None else D_F32
        p.bias_dtype = _dt_code(self.bias) if self.bias is not None else D_BF16
        p.group = int(self.group)
        p.N, p.K = int(self.N), int(self.K)
        p.num_slots = int(self.w.shape[0]) if slotted else 1
        p.reserved = 0
        self._keep = p
        return p


def dequant(P: OracleProj, slot: int = 0) -> np.ndarray:
    """fp32 [N, K] of one slot through the C per-element restatement."""
    out = np.empty((P.N, P.K), np.float32)
    lib().orc_dequant(ctypes.byref(P.c()), slot, out.ctypes.data)
    return out


def router_logits(x_bits: np.ndarray, G_bits: np.ndarray, bias_bits: Optional[np.ndarray] = None) -> np.ndarray:
    """bf16 router logits [T, R] in the GPU kernel's summation order (as fp32)."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    G = np.ascontiguousarray(G_bits, np.uint16)
    T, H = x.shape
    R = G.shape[0]
    out = np.empty((T, R), np.float32)
    b = np.ascontiguousarray(bias_bits, np.uint16) if bias_bits is not None else None
    lib().orc_router_logits(x.ctypes.data, T, H, G.ctypes.data, R, b.ctypes.data if b is not None else None,
                            out.ctypes.data)
    return out


def expert_forward(w13: OracleProj, w2: OracleProj, slot: int, x: np.ndarray, act: str = "silu",
                   alpha: float = 1.702, limit: float = 7.0, h_bf16: bool = True) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0]
    y = np.empty((M, w13.K), np.float64)
    rc = lib().orc_expert_forward(ctypes.byref(w13.c()), ctypes.byref(w2.c()), slot, x.ctypes.data, M, ACTS[act],
                                  alpha, limit, 1 if h_bf16 else 0, y.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"orc_expert_forward rc={rc}")
    return y


def moe_experts(w13: OracleProj, w2: OracleProj, x: np.ndarray, ids: np.ndarray, w: np.ndarray, *,
                E: int, slot_of_expert: Optional[np.ndarray] = None, act: str = "silu", alpha: float = 1.702,
                limit: float = 7.0, h_bf16: bool = True, on_input: bool = False, x_bf16: bool = True
                ) -> np.ndarray:
    """sum_j w[t,j] * expert_{ids[t,j]}(x[t]) in double, [T, H]."""
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    T, k = ids.shape
    out = np.empty((T, w13.K), np.float64)
    soe = np.ascontiguousarray(slot_of_expert, np.int32) if slot_of_expert is not None else None
    rc = lib().orc_moe_experts(ctypes.byref(w13.c()), ctypes.byref(w2.c()), soe.ctypes.data if soe is not None else None,
                               E, x.ctypes.data, T, k, ids.ctypes.data, w.ctypes.data, ACTS[act], alpha, limit,
                               1 if h_bf16 else 0, 1 if on_input else 0, 1 if x_bf16 else 0, out.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"orc_moe_experts rc={rc}")
    return out


# ----------------------------------------------------------------- whole layer
def layer_reference(spec: dict, x_bits: np.ndarray, *, ids: Optional[np.ndarray] = None,
                    w: Optional[np.ndarray] = None) -> dict:
    """Full MoE layer on bf16 input bits ``x_bits [T, H]``.

    ``spec`` keys: fmt, E, H, I, k, route_mode, renormalize, act, alpha, limit,
    w13 / w2 (:class:`OracleProj`), gate_w (bf16 bits [E, H]), gate_b (bits [E] or None),
    shared (dict w13/w2/gate bf16 bits, or None), slot_of_expert (or None).
    Returns logits [T, E], ids, w, out (float64 [T, H])."""
    x = bf16_bits_to_f32(x_bits)
    res = {}
    if ids is None:
        logits = router_logits(x_bits, spec["gate_w"], spec.get("gate_b"))
        ids, w = route(logits, spec["k"], spec["route_mode"], spec["renormalize"])
        res["logits"] = logits
    out = moe_experts(spec["w13"], spec["w2"], x, ids, w, E=spec["E"], slot_of_expert=spec.get("slot_of_expert"),
                      act=spec["act"], alpha=spec["alpha"], limit=spec["limit"])
    sh = spec.get("shared")
    if sh is not None:
        Is = sh["w2"].shape[1]
        sl = router_logits(x_bits, sh["gate"])  # [T, 1]
        sw = round_bf16(sigmoidf(sl))[:, 0]
        p13 = OracleProj("bf16", sh["w13"], 2 * Is, spec["H"])
        p2 = OracleProj("bf16", sh["w2"], spec["H"], Is)
        ys = expert_forward(p13, p2, 0, x, "silu")
        out = out + sw[:, None].astype(np.float64) * ys
        res["shared_w"] = sw
    res.update(ids=ids, w=w, out=out)
    return res


# ----------------------------------------------------------------- the reference's own CPU MoE
def ref_cpu_moe_available() -> bool:
    return os.path.exists(REF_LIB_PATH)


def ref_cpu_moe_forward_fast(x: np.ndarray, ids: np.ndarray, w: np.ndarray, gate_up: np.ndarray, down: np.ndarray,
                             threads: int = 0) -> np.ndarray:
    """Call freetoken_cpu_moe_forward_fast (cpu_moe.cpp:763-786) of the reference,
    built unmodified into oracle/_ref.  fp32 [T,H] x, int32 ids [T,k], fp32 w,
    gate_up [E, 2I, H] fp32, down [E, H, I] fp32."""
    L = ctypes.CDLL(REF_LIB_PATH)
    f = L.freetoken_cpu_moe_forward_fast
    f.restype = ctypes.c_int
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    f.argtypes = [vp, i32, i32, vp, vp, i32, vp, vp, i32, i32, vp, i32, i32, vp]
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    gate_up = np.ascontiguousarray(gate_up, np.float32)
    down = np.ascontiguousarray(down, np.float32)
    T, H = x.shape
    k = ids.shape[1]
    E, I2, _ = gate_up.shape
    out = np.zeros((T, H), np.float32)
    rc = f(x.ctypes.data, T, H, ids.ctypes.data, w.ctypes.data, k, gate_up.ctypes.data, down.ctypes.data, E, I2 // 2,
           None, int(threads), 0, out.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"freetoken_cpu_moe_forward_fast rc={rc}")
    return out


# ----------------------------------------------------------------- slot-pool LRU (pure Python)
@dataclass
class LruState:
    """OffloadMoeCache's bookkeeping (python/freetoken/moe/offload_cache.py:218-694):
    flat id = layer * E + expert."""
    L: int
    E: int
    S: int
    slot_for_id: list
    id_of_slot: list
    usage: list
    step: int = 0
    missing: int = 0
    calls: int = 0


def lru_new(L: int, E: int, S: int) -> LruState:
    return LruState(L, E, S, [-1] * (L * E), [-1] * S, [0] * S)


def lru_resync(st: LruState) -> None:
    """_resync_slot_for_id (offload_cache.py:401-435): slot_for_id rebuilt from id_of_slot."""
    st.slot_for_id = [-1] * (st.L * st.E)
    for s, i in enumerate(st.id_of_slot):
        if 0 <= i < st.L * st.E:
            st.slot_for_id[i] = s


def lru_ensure(st: LruState, layer_id: int, expert_ids) -> tuple:
    """ensure_experts (offload_cache.py:560-647), statement by statement: the
    routed experts in first-appearance order; step += 1; phase 1 stamps the
    slot of every resident one; phase 2 takes the missing ones in ascending id,
    each evicting ``min(range(S), key=(usage[s], s))`` and stamping it; then the
    resync.  Returns the plan ``(evict_slots, src_rows)``."""
    E, S, base = st.E, st.S, layer_id * st.E
    seen = []
    for e in expert_ids:
        e = int(e)
        if e not in seen:
            seen.append(e)
    step = st.step + 1
    st.step = step
    for e in seen:
        s = st.slot_for_id[base + e]
        if s != -1:
            st.usage[s] = step
    missing = sorted(e for e in seen if st.slot_for_id[base + e] == -1)
    st.missing += len(missing)
    st.calls += 1
    evict, src = [], []
    for e in missing:
        victim = min(range(S), key=lambda s: (st.usage[s], s))
        old = st.id_of_slot[victim]
        if old >= 0:
            st.slot_for_id[old] = -1
        st.id_of_slot[victim] = base + e
        st.slot_for_id[base + e] = victim
        st.usage[victim] = step
        evict.append(victim)
        src.append(e)
    lru_resync(st)
    return evict, src


def lru_ensure_chunk(st: LruState, layer_id: int, expert_ids, chunk: int, cap: int) -> tuple:
    """The chunked decode step of this build's moe_offload_forward (not in the
    reference): the distinct routed experts (ids >= 0) in ascending id, ranks
    [chunk * cap, (chunk + 1) * cap) through :func:`lru_ensure`; chunk 0 is
    always a call (an empty one still steps, as the reference's does), a later
    empty chunk leaves the state alone.  Returns ``(plan or None, members)``."""
    uniq = sorted({int(e) for e in expert_ids if int(e) >= 0})
    members = uniq[chunk * cap:(chunk + 1) * cap]
    if not members and chunk > 0:
        return None, members
    return lru_ensure(st, layer_id, members), members
