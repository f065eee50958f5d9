"""ctypes binding of ``libftmoe.so`` (the gfx950 HIP kernels behind the C ABI
declared in ``include/ftmoe.h``).

The library is built in-tree by ``freetoken-intel_amd/csrc/Makefile``
(``__graft_entry__.build()``).  There is deliberately no fallback: every
product entry point raises when the library is missing or a tensor is not on
the GPU.  The ctypes/``.so`` loading pattern mirrors the reference's CPU MoE
binding (python/freetoken/kernel/cpu_moe.py:195-245), minus its JIT compiler.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_native", "libftmoe.so")

# ---- constants (include/ftmoe.h) -------------------------------------------
ABI_VERSION = 1
OK = 0
ERR_NULL = -1
ERR_DIM = -2
ERR_FORMAT = -3
ERR_HIP = -4
ERR_WORKSPACE = -5
ERR_ALIGN = -6
ERR_HANDLE = -100

FMT_BF16 = 0
FMT_FP8_BLOCK = 1
FMT_GPTQ_INT4 = 2
FMT_INT8_PACKED = 3
FMT_MXFP4 = 4
FMT_FP32 = 5
FMT_FP8_E5M2_BLOCK = 6

DT_F32 = 0
DT_F16 = 1
DT_BF16 = 2

ROUTE_SOFTMAX_TOPK = 0
ROUTE_SOFTMAX_TOPK_LOWP = 1
ROUTE_TOPK_SOFTMAX = 2

ACT_SILU = 0
ACT_GELU = 1
ACT_RELU = 2
ACT_SWIGLU_OAI = 3

WS_CTRL_BYTES = 4096
NOALLOC_SCRATCH_BYTES = 16 << 20
WS_ERROR_OFFSET = 12
WS_ERR_SLOT = 1
WS_ERR_ID = 2
WS_ERR_LIST = 4

PROJ_RING_B = 1  # ftm_proj.flags: FP8 stage B on the ring tile (FTM_PROJ_RING_B)
STAGE_ROUTER = 0
STAGE_TOPK = 1
STAGE_W13 = 2
STAGE_W2 = 3
STAGE_COMBINE = 4

_ERR_TEXT = {
    ERR_NULL: "a required pointer is NULL",
    ERR_DIM: "a dimension is out of range or inconsistent",
    ERR_FORMAT: "unsupported format / dtype / mode combination",
    ERR_HIP: "a HIP runtime call failed",
    ERR_WORKSPACE: "workspace missing or too small",
    ERR_ALIGN: "a pointer or stride is not 16-byte aligned",
    ERR_HANDLE: "unknown handle",
}


class FtmProj(ctypes.Structure):
    """``ftm_proj``: one projection bank ([slots, N, K] logical)."""

    _fields_ = [
        ("w", ctypes.c_void_p),
        ("s", ctypes.c_void_p),
        ("z", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("w_stride", ctypes.c_int64),
        ("s_stride", ctypes.c_int64),
        ("z_stride", ctypes.c_int64),
        ("bias_stride", ctypes.c_int64),
        ("fmt", ctypes.c_int32),
        ("s_dtype", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("num_slots", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


class FtmMoeLayer(ctypes.Structure):
    """``ftm_moe_layer``: routed banks, router, activation, shared expert."""

    _fields_ = [
        ("w13", FtmProj),
        ("w2", FtmProj),
        ("slot_of_expert", ctypes.c_void_p),
        ("gate_w", ctypes.c_void_p),
        ("gate_b", ctypes.c_void_p),
        ("shared_w13", ctypes.c_void_p),
        ("shared_w2", ctypes.c_void_p),
        ("shared_gate", ctypes.c_void_p),
        ("num_experts", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("topk", ctypes.c_int32),
        ("shared_inter", ctypes.c_int32),
        ("route_mode", ctypes.c_int32),
        ("renormalize", ctypes.c_int32),
        ("act", ctypes.c_int32),
        ("swiglu_alpha", ctypes.c_float),
        ("swiglu_limit", ctypes.c_float),
        ("apply_router_weight_on_input", ctypes.c_int32),
        ("act_dtype", ctypes.c_int32),
        ("h_dtype", ctypes.c_int32),
    ]


# Every symbol include/ftmoe.h declares (tests check the export table against this).
EXPORTED = (
    "ftm_version",
    "ftm_moe_workspace_bytes",
    "ftm_workspace_init",
    "ftm_moe_forward",
    "ftm_moe_forward_noalloc",
    "ftm_moe_forward_stage",
    "ftm_moe_stage_kernel",
    "ftm_moe_forward_routed",
    "ftm_route",
    "ftm_linear",
    "ftm_expert_forward",
    "ftm_dequant",
    "ftm_lru_ensure",
    "ftm_lru_materialize",
    "ftm_copy_slots",
    "ftm_lru_ensure_dev",
    "ftm_copy_slots_dev",
    "ftm_cpu_moe_forward",
    "ftm_cpu_moe_submit",
    "ftm_cpu_moe_wait",
    "ftm_cpu_avx512",
)


class FtmBankCopy(ctypes.Structure):
    """``ftm_bank_copy`` (include/ftmoe.h)."""
    _fields_ = [
        ("host_bank", ctypes.c_void_p),
        ("dev_pool", ctypes.c_void_p),
        ("row_bytes", ctypes.c_int64),
    ]

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load ``libftmoe.so`` once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() "
            "(make -C freetoken-intel_amd/csrc). ftmoe has no CPU fallback."
        )
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    P_proj = ctypes.POINTER(FtmProj)
    P_layer = ctypes.POINTER(FtmMoeLayer)
    L.ftm_version.restype = ctypes.c_int
    L.ftm_version.argtypes = []
    L.ftm_moe_workspace_bytes.restype = sz
    L.ftm_moe_workspace_bytes.argtypes = [P_layer, i32]
    L.ftm_workspace_init.restype = ctypes.c_int
    L.ftm_workspace_init.argtypes = [vp, sz, vp]
    L.ftm_moe_forward.restype = ctypes.c_int
    L.ftm_moe_forward.argtypes = [P_layer, vp, i32, vp, vp, vp, vp, vp, sz, vp]
    L.ftm_moe_forward_noalloc.restype = ctypes.c_int
    L.ftm_moe_forward_noalloc.argtypes = [P_layer, vp, i32, vp, vp, vp, vp, vp]
    L.ftm_moe_forward_stage.restype = ctypes.c_int
    L.ftm_moe_forward_stage.argtypes = [P_layer, vp, i32, vp, i32, vp, sz, vp]
    L.ftm_moe_stage_kernel.restype = ctypes.c_char_p
    L.ftm_moe_stage_kernel.argtypes = [P_layer, i32, i32]
    L.ftm_moe_forward_routed.restype = ctypes.c_int
    L.ftm_moe_forward_routed.argtypes = [P_layer, vp, i32, vp, vp, vp, vp, sz, vp]
    L.ftm_route.restype = ctypes.c_int
    L.ftm_route.argtypes = [P_layer, vp, i32, vp, i32, vp, vp, vp, vp, sz, vp]
    L.ftm_linear.restype = ctypes.c_int
    L.ftm_linear.argtypes = [P_proj, i32, vp, i32, i32, vp, i32, vp, i32, i32, vp]
    L.ftm_expert_forward.restype = ctypes.c_int
    L.ftm_expert_forward.argtypes = [P_layer, i32, vp, i32, vp, vp, sz, vp]
    L.ftm_dequant.restype = ctypes.c_int
    L.ftm_dequant.argtypes = [P_proj, i32, vp, i32, i32, vp]
    L.ftm_lru_ensure.restype = ctypes.c_int
    L.ftm_lru_ensure.argtypes = [i32, i32, i32, i32, vp, i32, vp, vp, vp, vp, vp, vp, vp]
    L.ftm_lru_materialize.restype = ctypes.c_int
    L.ftm_lru_materialize.argtypes = [i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]
    L.ftm_copy_slots.restype = ctypes.c_int
    L.ftm_copy_slots.argtypes = [vp, vp, i64, vp, vp, i32, vp, vp]
    L.ftm_lru_ensure_dev.restype = ctypes.c_int
    L.ftm_lru_ensure_dev.argtypes = [i32, i32, i32, i32, vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                     vp]
    L.ftm_copy_slots_dev.restype = ctypes.c_int
    L.ftm_copy_slots_dev.argtypes = [ctypes.POINTER(FtmBankCopy), i32, i32, i32, vp, vp, vp, i32, vp]
    L.ftm_cpu_moe_forward.restype = ctypes.c_int
    L.ftm_cpu_moe_forward.argtypes = [P_layer, vp, i32, vp, vp, vp, i32, i32, vp]
    L.ftm_cpu_moe_submit.restype = ctypes.c_int64
    L.ftm_cpu_moe_submit.argtypes = [P_layer, vp, i32, vp, vp, vp, i32, vp]
    L.ftm_cpu_moe_wait.restype = ctypes.c_int
    L.ftm_cpu_moe_wait.argtypes = [i64]
    L.ftm_cpu_avx512.restype = ctypes.c_int
    L.ftm_cpu_avx512.argtypes = []
    _lib = L
    return L


class FtmError(RuntimeError):
    def __init__(self, what: str, code: int):
        super().__init__(f"{what} failed with code {code}: {_ERR_TEXT.get(code, 'unknown error')}")
        self.code = code


def check(rc: int, what: str) -> int:
    if rc < 0:
        raise FtmError(what, rc)
    return rc


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.float32:
        return DT_F32
    if dtype == torch.float16:
        return DT_F16
    if dtype == torch.bfloat16:
        return DT_BF16
    raise TypeError(f"unsupported dtype {dtype} (expected float32, float16 or bfloat16)")


def require_gpu(t, name: str) -> None:
    """The product path runs only on the GPU: refuse CPU tensors loudly."""
    if t is not None and not t.is_cuda:
        raise RuntimeError(
            f"{name} must be a ROCm device tensor: ftmoe runs only as gfx950 HIP kernels (no CPU fallback)"
        )


def stream_of(t) -> int:
    import torch

    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()
