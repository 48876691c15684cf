"""lumen_amd: lumen's compiled-graph hot path on AMD Instinct MI355X (gfx950).

``lumen_amd.compile(fn, device="hip")`` traces ``fn`` into lumen's strict-primitive graph, runs the hip
pass pipeline over it and executes it as one static plan in one device workspace, with hand-written
CDNA4 kernels (``libnhip.so``, C ABI in ``include/nhip.h``) and generated fused loop kernels.
"""

from lumen_amd import autograd, autotune, functional, nn
from lumen_amd.autograd import grad, value_and_grad, vjp
from lumen_amd.config import config
from lumen_amd.graph import prims
from lumen_amd.graph.compiled import Compiled, compile
from lumen_amd.graph.trace import make_graph
from lumen_amd.tensor import Tensor, empty, from_numpy, full, ones, tensor, to_numpy, zeros

bool = "bool"
uint8, uint16, uint32, uint64 = "uint8", "uint16", "uint32", "uint64"
int8, int16, int32, int64 = "int8", "int16", "int32", "int64"
float16, bfloat16, float32, float64 = "float16", "bfloat16", "float32", "float64"

__all__ = [
    "Compiled", "Tensor", "autograd", "autotune", "compile", "config", "empty", "from_numpy", "full", "functional", "grad",
    "make_graph", "nn", "ones", "prims", "tensor", "to_numpy", "value_and_grad", "vjp", "zeros",
]
