"""Hybrid CPU-offload executor: hot experts on the GPU, cold experts on host
threads (C ABI ``mi_moe_hybrid_*``, include/mi_moe.h).

The reference runs the whole layer in a host callback between copies
(``moe_forward_npu_stream``, Int8-gemm/nanovllm_ops.cpp:244-305) and plans the
per-expert split (README.md:124-134).  Usage::

    hm = HybridMoE(E, H, I, quant_type, host_experts=[5, 17, 99])
    hm.store_awq(w13_q, w13_z, w13_s, w2_q, w2_z, w2_s)   # all E experts, host or HIP tensors
    y = hm.forward(hidden, topk_ids, topk_w)              # HIP tensors, current stream

Only the hot experts' weights reach device memory.  ``host_forward`` runs the
cold experts alone on host tensors (fp32 partial), synchronously.
"""
from __future__ import annotations

import ctypes

__all__ = ["HybridMoE"]


class HybridMoE:
    def __init__(self, num_experts: int, hidden: int, intermediate: int, quant_type: int,
                 host_experts, num_threads: int = 0):
        from . import capi, check
        self._L = capi()
        self.E, self.H, self.I, self.quant = num_experts, hidden, intermediate, quant_type
        mask = (ctypes.c_uint8 * num_experts)()
        for e in host_experts:
            if not 0 <= int(e) < num_experts:
                raise ValueError(f"host expert {e} out of range [0, {num_experts})")
            mask[int(e)] = 1
        self._h = ctypes.c_void_p()
        check(self._L.mi_moe_hybrid_create(num_experts, hidden, intermediate, quant_type, mask, num_threads,
                                           ctypes.byref(self._h)), "mi_moe_hybrid_create")

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            self._L.mi_moe_hybrid_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _src(tensors):
        on_dev = {t.is_cuda for t in tensors}
        if len(on_dev) != 1:
            raise ValueError("weights must all be host tensors or all HIP tensors")
        return [t.contiguous() for t in tensors], int(on_dev.pop())

    def _stream(self, on_dev):
        from . import stream_ptr
        return stream_ptr() if on_dev else None

    def store_quantized(self, gate_up_qs, gate_up_d, down_qs, down_d):
        import torch
        from . import check, dtype_code
        (a, b, c, d), on_dev = self._src([gate_up_qs, gate_up_d, down_qs, down_d])
        if b.dtype != d.dtype:
            raise TypeError("gate_up_d and down_d must share one dtype")
        check(self._L.mi_moe_hybrid_store_quantized(self._h, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                                    d.data_ptr(), dtype_code(b.dtype), on_dev,
                                                    self._stream(on_dev)), "mi_moe_hybrid_store_quantized")
        if on_dev:
            torch.cuda.synchronize()

    def store_awq(self, w13_q, w13_z, w13_s, w2_q, w2_z, w2_s, group: int = 128):
        import torch
        from . import check, dtype_code
        ts, on_dev = self._src([w13_q, w13_z, w13_s, w2_q, w2_z, w2_s])
        check(self._L.mi_moe_hybrid_store_awq(self._h, *[t.data_ptr() for t in ts], group,
                                              dtype_code(ts[2].dtype), on_dev, self._stream(on_dev)),
              "mi_moe_hybrid_store_awq")
        if on_dev:
            torch.cuda.synchronize()

    def _check_shapes(self, hidden, topk_ids, topk_w):
        """The C ABI trusts T, H and K; mismatched tensors are rejected here
        (the same rules as the torch op, nanovllm_shim.cpp forward_into)."""
        import torch
        if hidden.dim() != 2 or topk_ids.dim() != 2 or topk_w.dim() != 2:
            raise ValueError("expected hidden [T,H], topk_ids [T,K], topk_w [T,K]")
        if hidden.shape[1] != self.H:
            raise ValueError(f"hidden size {hidden.shape[1]} != handle H {self.H}")
        if topk_ids.shape[0] != hidden.shape[0] or topk_w.shape[0] != hidden.shape[0]:
            raise ValueError("topk_ids / topk_w rows must equal the token count of hidden")
        if topk_w.shape[1] != topk_ids.shape[1]:
            raise ValueError("topk_ids and topk_w must have the same top_k")
        if hidden.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError(f"hidden must be float16 or bfloat16, got {hidden.dtype}")

    def forward(self, hidden, topk_ids, topk_w, out=None):
        import torch
        from . import check, dtype_code, stream_ptr
        if not (hidden.is_cuda and topk_ids.is_cuda and topk_w.is_cuda):
            raise ValueError("forward takes HIP tensors; host_forward runs the cold experts on host tensors")
        self._check_shapes(hidden, topk_ids, topk_w)
        if topk_ids.device != hidden.device or topk_w.device != hidden.device:
            raise ValueError("hidden, topk_ids and topk_w must be on the same device")
        if out is not None and (out.shape != hidden.shape or out.dtype != hidden.dtype
                                or out.device != hidden.device or not out.is_contiguous()):
            raise ValueError("out must be a contiguous tensor with hidden's shape, dtype and device")
        x = hidden.contiguous()
        ids = topk_ids.to(torch.int32).contiguous()
        w = topk_w.to(torch.float32).contiguous()
        y = torch.empty_like(x) if out is None else out
        check(self._L.mi_moe_hybrid_forward(self._h, x.data_ptr(), y.data_ptr(), w.data_ptr(), ids.data_ptr(),
                                            x.shape[0], ids.shape[1], dtype_code(x.dtype), stream_ptr()),
              "mi_moe_hybrid_forward")
        return y

    def host_forward(self, hidden, topk_ids, topk_w):
        import torch
        from . import check, dtype_code
        self._check_shapes(hidden, topk_ids, topk_w)
        x = hidden.detach().cpu().contiguous()
        ids = topk_ids.detach().cpu().to(torch.int32).contiguous()
        w = topk_w.detach().cpu().to(torch.float32).contiguous()
        y = torch.empty(x.shape[0], self.H, dtype=torch.float32)
        check(self._L.mi_moe_hybrid_host_forward(self._h, x.data_ptr(), w.data_ptr(), ids.data_ptr(), x.shape[0],
                                                 ids.shape[1], dtype_code(x.dtype), y.data_ptr()),
              "mi_moe_hybrid_host_forward")
        return y

    def stats(self) -> dict:
        from . import check
        dev, host, hb, pairs = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        ms, qms = ctypes.c_double(), ctypes.c_double()
        check(self._L.mi_moe_hybrid_get_stats(self._h, ctypes.byref(dev), ctypes.byref(host), ctypes.byref(hb),
                                              ctypes.byref(ms), ctypes.byref(pairs), ctypes.byref(qms)),
              "mi_moe_hybrid_get_stats")
        return {"device_experts": dev.value, "host_experts": host.value, "host_weight_bytes": hb.value,
                "last_host_ms": ms.value, "last_host_pairs": pairs.value, "last_queue_ms": qms.value}
