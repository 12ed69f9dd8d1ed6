"""mlx-hip: an MI355X (gfx950) compute backend for the oxidizedMLX tensor runtime.

The product is ``libmlxhip.so`` (HIP kernels + C ABI, include/mlxhip.h). This
package is its Python face: ctypes bindings (``abi``), the OpKind/TensorMeta
mirror (``opkind``), and the host-side Backend/Stream wrappers (``backend``).
"""
from . import abi  # noqa: F401
from .opkind import NodeInput, Op, OpKind, TensorMeta, meta  # noqa: F401
