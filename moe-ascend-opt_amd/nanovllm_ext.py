"""Drop-in module name of the reference extension (``import nanovllm_ext``,
Int8-gemm/test/fused_moe_cpu.py:7): importing it registers
torch.classes.nanovllm.MoEInfer and torch.ops.nanovllm.moe_forward backed by
the MI355X kernels of libmimoe.so."""
import nanovllm_moe as _m

_m.load()
