"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every entry point include/mi_moe.h declares; the torch shim registers the
reference schema (Int8-gemm/nanovllm_ops.cpp:349-412); argument errors come
back as status codes with a message (no compute without a GPU)."""
import ctypes
import os
import re

import torch

import nanovllm_moe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "mi_moe.h")).read()
    return sorted(set(re.findall(r"\b(mi_moe_[a-z0-9_]+)\s*\(", src)))


def test_header_and_symbol_list_agree():
    assert _declared() == sorted(nanovllm_moe.C_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(nanovllm_moe.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    L = nanovllm_moe.capi()
    assert L.mi_moe_version() >= 100


def test_shim_registers_reference_schema():
    nanovllm_moe.load()
    import nanovllm_ext  # noqa: F401  (drop-in module name)
    schema = str(torch.ops.nanovllm.moe_forward.default._schema)
    assert schema.startswith("nanovllm::moe_forward(Tensor hidden, Tensor topk_ids, Tensor topk_w, "
                             "__torch__.torch.classes.nanovllm.MoEInfer moe) -> Tensor")
    assert "Tensor(a!) out" in str(torch.ops.nanovllm.moe_forward_out.default._schema)
    assert "(Tensor, Tensor)" in str(torch.ops.nanovllm.moe_topk_softmax.default._schema)
    assert "router_logits" in str(torch.ops.nanovllm.moe_forward_logits.default._schema)
    methods = {str(s).split("(")[0] for s in torch._C._jit_get_custom_class_schemas()
               if "nanovllm.MoEInfer" in str(s)}
    for m in ("__init__", "quantize_and_store_expert", "store_quantized_repack", "store_awq_repack",
              "get_last_run_time_ms", "get_quant_type", "get_num_experts",
              "get_hidden_size", "get_intermediate_size"):
        assert m in methods, m


def test_argument_errors_are_status_codes():
    L = nanovllm_moe.capi()
    P = ctypes.c_void_p
    h = P()
    assert L.mi_moe_create(0, 2048, 768, 2, ctypes.byref(h)) == 1
    assert b"positive" in L.mi_moe_last_error()
    assert L.mi_moe_create(8, 2048, 768, 7, ctypes.byref(h)) == 1
    assert L.mi_moe_create(8, 2000, 768, 0, ctypes.byref(h)) == 1
    assert b"multiple of 32" in L.mi_moe_last_error()
    assert L.mi_moe_create(8, 2048, 768, 2, None) == 1
    assert L.mi_moe_forward(None, None, None, None, None, 1, 8, 1, None) == 1
    assert b"null handle" in L.mi_moe_last_error()
    assert L.mi_moe_route(None, -1, 8, 128, None, None, None, None, None) == 1
    assert L.mi_moe_quantize_act_q8_0(None, 1, 1, 33, None, None, None) == 1
    assert L.mi_moe_topk_softmax(None, 3, 1, 128, 8, 1, None, None, None) == 1      # dtype
    assert L.mi_moe_topk_softmax(None, 2, 1, 600, 8, 1, None, None, None) == 1      # E > 512
    assert L.mi_moe_topk_softmax(None, 2, 1, 8, 9, 1, None, None, None) == 1        # K > E
    assert b"top_k" in L.mi_moe_last_error()
    assert L.mi_moe_topk_softmax(None, 2, 0, 128, 8, 1, None, None, None) == 0      # T = 0: nothing
    assert L.mi_moe_forward_logits(None, None, None, None, 2, 1, 8, 1, 1, None, None, None) == 1
    assert b"null handle" in L.mi_moe_last_error()
    assert L.mi_moe_destroy(None) == 0
    assert L.mi_moe_get_last_run_time_ms(None) < 0


def test_create_rejects_shapes_no_path_serves():
    """Without a GPU the LDS limit is 64 KB: a W4A16 handle whose grouped GEMMs
    do not fit (DeepSeek-like H = 7168: 71,424 B for gate_up) is refused with
    EUNSUPPORTED at create time; shapes that fit are accepted by the shape
    rules (create then fails only for want of a HIP device)."""
    L = nanovllm_moe.capi()
    h = ctypes.c_void_p()
    assert L.mi_moe_create(8, 7168, 2048, 2, ctypes.byref(h)) == 3
    assert b"LDS" in L.mi_moe_last_error()
    assert L.mi_moe_create(8, 2048, 768, 2, ctypes.byref(h)) in (0, 4)
    if h.value:
        L.mi_moe_destroy(h)
