"""hkmoe -- MI355X (gfx950) FP8 mixture-of-experts grouped-GEMM path.

Host-side Python layer over the ``tk_kernel`` pybind11 module, which in turn
wraps the C ABI of ``libhkmoe.so`` (include/hkmoe.h).  All compute runs in the
hand-written HIP kernels of that library; there is no CPU or PyTorch fallback:
importing this package raises ImportError when the native module is missing.

Entry points
  tk_kernel.dispatch_*      raw kernel entry points (reference calling style:
                            positional, caller-allocated torch tensors)
  hkmoe.MoELayer            owns e4m3 expert weights + scales, allocates the
                            workspace once per token count, runs the layer
  hkmoe.moe_forward_steps   the same layer one kernel at a time, returning
                            every intermediate (for parity tests)
  hkmoe.quant_*             device quantisers (per-tensor, 1x128, 128x128)
"""
import os
import sys

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG_ROOT not in sys.path:
    sys.path.insert(0, _PKG_ROOT)

try:
    import tk_kernel  # noqa: E402
except ImportError as exc:  # pragma: no cover - exercised only on a broken tree
    raise ImportError(
        "hkmoe: native module tk_kernel is not built; run "
        "`python distributed-hipkittens_amd/hkmoe/build.py` (or __graft_entry__.build())"
    ) from exc

from .layer import (MoELayer, moe_forward, moe_forward_steps, pack_weights,  # noqa: E402
                    quant_block, quant_group, quant_tensor, gemm_fp8, quant_mx, mx_pack_scales, gemm_mx,
                    mx_pack_weight_scales, moe_forward_mx_steps, MoELayerMX)

LIB_PATH = os.path.join(_PKG_ROOT, "libhkmoe.so")
SCALE_TENSOR = tk_kernel.SCALE_TENSOR
SCALE_BLOCK = tk_kernel.SCALE_BLOCK

__all__ = ["tk_kernel", "MoELayer", "moe_forward", "moe_forward_steps", "pack_weights", "quant_block",
           "quant_group", "quant_tensor", "gemm_fp8", "quant_mx", "mx_pack_scales", "gemm_mx",
           "mx_pack_weight_scales", "moe_forward_mx_steps", "MoELayerMX", "LIB_PATH",
           "SCALE_TENSOR", "SCALE_BLOCK"]
