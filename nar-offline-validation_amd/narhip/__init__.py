"""narhip: MI355X-native kernels for NAR's online rotate-and-quantize path.

Operators (all on the GPU, all through libnarhip.so, registered with the
torch dispatcher as torch.ops.narhip.* by narhip/library.py):
  ops.rotate_quant     fused Kronecker/block Hadamard + rank-k + INT4 quantize
  ops.rank_projection  split rank-k projection partials (Kernel A)
  ops.group_quant      rotate + rank-k from partials + quantize (Kernel B)
  ops.transform_f16    E28's fp16 transform
  ops.dequantize       packed INT4 -> fp32
  ops.w4a4_gemm        group-asymmetric INT4 x INT4 GEMM
  hooks.*              dynamic_asym_int4, full_hadamard_rows and the fused form
The drop-in modules for the reference's Python call sites live beside this
package: nar/kernels/r4_fused_v2.py, nar/kernels/r4_fused_v3.py and
nar_r4_kernel.py.
"""

from . import library, ops  # noqa: F401
from ._lib import LIB_PATH, load  # noqa: F401

__all__ = ["library", "ops", "load", "LIB_PATH"]
