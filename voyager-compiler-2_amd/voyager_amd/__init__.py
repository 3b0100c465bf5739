"""MI355X-native (gfx950) execution of Voyager's quantized-operator path.

The ``quantized_ops`` kernels launch the HIP library ``_lib/libvoyager_hip.so``
through its C ABI (``include/voyager_hip.h``).  Importing the package
registers nothing:

* ``import voyager_amd.library`` defines the ``quantized_ops`` namespace
  standalone (the reference's schema strings) with these kernels bound;
* ``voyager_amd.kernels.register(lib)`` binds them onto a namespace another
  library defined -- the reference's ``quantized_ops_lib``.
"""

from . import _lib, formats  # noqa: F401

__all__ = ["formats"]
