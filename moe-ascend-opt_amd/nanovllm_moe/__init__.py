"""MI355X-native fused-MoE expert library (gfx950), drop-in for the reference's
``nanovllm_ext`` extension (Int8-gemm/nanovllm_ops.cpp:349-412).

After ``nanovllm_moe.load()`` (or ``import nanovllm_ext``):

    h = torch.classes.nanovllm.MoEInfer(E, H, I, quant_type)   # 0 Q8_0, 1 Q4_0, 2 W4A16
    h.store_quantized_repack(gate_up_qs, gate_up_d, down_qs, down_d)   # Q8_0 / Q4_0
    h.store_awq_repack(w13_q, w13_z, w13_s, w2_q, w2_z, w2_s, 128)      # W4A16
    y = torch.ops.nanovllm.moe_forward(hidden, topk_ids, topk_w, h)     # HIP tensors

The op dispatches on the tensors' device, like the reference's registration
(Int8-gemm/nanovllm_ops.cpp:410-412).  HIP tensors run the hand-written HIP
kernels of ``libmimoe.so`` on the current stream; a missing library raises,
and the HIP key never falls back to the host.  CPU tensors run the reference
CPU algorithm on host cores (the CPU key: Q8_0 / Q4_0 on the host engine,
W4A16 on the host executor), from the host copy of the weights a handle keeps
when no HIP device is present or MIMOE_HOST_WEIGHTS=1.
"""
from __future__ import annotations

import ctypes
import os

from . import formats  # noqa: F401
from .hybrid import HybridMoE  # noqa: F401

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmimoe.so")
SHIM_PATH = os.path.join(PKG_DIR, "libnanovllm_shim.so")

Q8_0, Q4_0, W4A16 = 0, 1, 2
F16, BF16, F32 = 0, 1, 2   # dtype codes (F32: router logits only)

_loaded = False
_capi = None

# exported C-ABI symbols (include/mi_moe.h)
C_SYMBOLS = (
    "mi_moe_last_error", "mi_moe_version", "mi_moe_create", "mi_moe_destroy",
    "mi_moe_get_info", "mi_moe_store_quantized", "mi_moe_quantize_and_store_expert",
    "mi_moe_store_awq", "mi_moe_forward", "mi_moe_forward_noalloc", "mi_moe_get_last_run_time_ms",
    "mi_moe_set_timing", "mi_moe_reserve", "mi_moe_quantize_act_q8_0", "mi_moe_route", "mi_moe_block_dots",
    "mi_moe_block_dots_mfma",
    "mi_moe_get_last_phase_times_ms", "mi_moe_topk_softmax", "mi_moe_forward_logits",
    "mi_moe_hybrid_create", "mi_moe_hybrid_destroy", "mi_moe_hybrid_store_quantized",
    "mi_moe_hybrid_store_awq", "mi_moe_hybrid_forward", "mi_moe_hybrid_host_forward",
    "mi_moe_hybrid_get_stats", "mi_moe_cpu_create", "mi_moe_cpu_destroy", "mi_moe_cpu_store_quantized",
    "mi_moe_cpu_quantize_and_store_expert", "mi_moe_cpu_forward", "mi_moe_cpu_get_info", "mi_moe_cpu_set_isa",
    "mi_moe_cpu_isa_name", "mi_moe_cpu_topk_softmax", "mi_moe_cpu_create_numa",
)


class NativeLibraryMissing(RuntimeError):
    pass


def load():
    """Register torch.classes.nanovllm.MoEInfer / torch.ops.nanovllm.* (idempotent)."""
    global _loaded
    if _loaded:
        return True
    import torch  # noqa: F401  (the HIP runtime must come from torch's process image)
    if not (os.path.exists(SHIM_PATH) and os.path.exists(LIB_PATH)):
        raise NativeLibraryMissing(
            f"native library not built ({SHIM_PATH}); run "
            "`python moe-ascend-opt_amd/nanovllm_moe/build.py` or __graft_entry__.build()")
    torch.ops.load_library(SHIM_PATH)
    _loaded = True
    return True


def capi():
    """ctypes view of libmimoe.so (the C ABI), with argtypes declared."""
    global _capi
    if _capi is not None:
        return _capi
    import torch  # noqa: F401
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(f"{LIB_PATH} not built")
    L = ctypes.CDLL(LIB_PATH)
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    L.mi_moe_last_error.restype = ctypes.c_char_p
    L.mi_moe_last_error.argtypes = []
    L.mi_moe_version.restype = I
    L.mi_moe_create.argtypes = [I64, I64, I64, I, ctypes.POINTER(P)]
    L.mi_moe_destroy.argtypes = [P]
    L.mi_moe_get_info.argtypes = [P, P, P, P, P, P]
    L.mi_moe_store_quantized.argtypes = [P, P, P, P, P, I, I, P]
    L.mi_moe_quantize_and_store_expert.argtypes = [P, I64, I, P, I, I, P]
    L.mi_moe_store_awq.argtypes = [P, P, P, P, P, P, P, I64, I, I, P]
    L.mi_moe_forward.argtypes = [P, P, P, P, P, I64, I64, I, P]
    L.mi_moe_forward_noalloc.argtypes = [P, P, P, P, P, I64, I64, I, P]
    L.mi_moe_get_last_run_time_ms.restype = ctypes.c_double
    L.mi_moe_get_last_run_time_ms.argtypes = [P]
    L.mi_moe_set_timing.argtypes = [P, I]
    L.mi_moe_reserve.argtypes = [P, I64, I64, P]
    L.mi_moe_get_last_phase_times_ms.argtypes = [P, ctypes.POINTER(ctypes.c_double), I]
    L.mi_moe_quantize_act_q8_0.argtypes = [P, I, I64, I64, P, P, P]
    L.mi_moe_route.argtypes = [P, I64, I64, I64, P, P, P, P, P]
    L.mi_moe_block_dots.argtypes = [P, I64, I, P, I64, P, P]
    L.mi_moe_block_dots_mfma.argtypes = [P, I64, I, P, I64, P, P, P]
    L.mi_moe_topk_softmax.argtypes = [P, I, I64, I64, I64, I, P, P, P]
    L.mi_moe_forward_logits.argtypes = [P, P, P, P, I, I64, I64, I, I, P, P, P]
    L.mi_moe_hybrid_create.argtypes = [I64, I64, I64, I, P, I, ctypes.POINTER(P)]
    L.mi_moe_hybrid_destroy.argtypes = [P]
    L.mi_moe_hybrid_store_quantized.argtypes = [P, P, P, P, P, I, I, P]
    L.mi_moe_hybrid_store_awq.argtypes = [P, P, P, P, P, P, P, I64, I, I, P]
    L.mi_moe_hybrid_forward.argtypes = [P, P, P, P, P, I64, I64, I, P]
    L.mi_moe_hybrid_host_forward.argtypes = [P, P, P, P, I64, I64, I, P]
    L.mi_moe_hybrid_get_stats.argtypes = [P, P, P, P, P, P, P]
    L.mi_moe_cpu_create.argtypes = [I64, I64, I64, I, I, I, ctypes.POINTER(P)]
    L.mi_moe_cpu_destroy.argtypes = [P]
    L.mi_moe_cpu_store_quantized.argtypes = [P, P, P, P, P, I]
    L.mi_moe_cpu_quantize_and_store_expert.argtypes = [P, I64, I, P, I]
    L.mi_moe_cpu_forward.argtypes = [P, P, P, P, P, I64, I64, I]
    L.mi_moe_cpu_get_info.argtypes = [P, P, P, P, P, P, P]
    L.mi_moe_cpu_set_isa.argtypes = [P, I]
    L.mi_moe_cpu_topk_softmax.argtypes = [P, I64, I64, I64, I, P, P]
    L.mi_moe_cpu_create_numa.argtypes = [I64, I64, I64, I, I, I, ctypes.POINTER(P)]
    L.mi_moe_cpu_isa_name.restype = ctypes.c_char_p
    L.mi_moe_cpu_isa_name.argtypes = [I]
    for name in C_SYMBOLS:
        fn = getattr(L, name)
        if fn.restype is ctypes.c_int or fn.restype is None:
            if name not in ("mi_moe_last_error", "mi_moe_get_last_run_time_ms", "mi_moe_cpu_isa_name"):
                fn.restype = I
    _capi = L
    return L


def check(rc: int, what: str = "mi_moe"):
    if rc != 0:
        msg = capi().mi_moe_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (status {rc})")


def stream_ptr(device=None):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dt) -> int:
    import torch
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    raise TypeError(f"unsupported dtype {dt}")
