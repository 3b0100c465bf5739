"""MI355X-native (gfx950) execution of Voyager's quantized-operator path.

Importing the package registers the ``quantized_ops`` torch.library namespace
(``voyager_amd.ops``) whose CUDA-key kernels launch the HIP library
``_lib/libvoyager_hip.so`` through its C ABI (``include/voyager_hip.h``).
"""

from . import _lib, formats, ops  # noqa: F401  (ops registers the library)
from . import gemm, packed  # noqa: F401  (gemm registers the GEMM ops)
from . import conv, decode, sparse  # noqa: F401  (conv and sparse register their ops)

__all__ = ["conv", "decode", "formats", "gemm", "ops", "packed", "sparse"]
