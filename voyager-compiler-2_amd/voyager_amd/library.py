"""The standalone ``quantized_ops`` namespace.

Importing this module defines ``quantized_ops`` with the reference's schema
strings (``voyager_amd.schemas``), binds the package's CUDA and fake kernels
to it (``voyager_amd.kernels.register``) and registers the accelerator-layout
twins as torch restatements.  Use it where the reference is not loaded (the
GPU box, the tests, the bench); where the reference defines the namespace
itself, bind the kernels onto its library with
``voyager_amd.kernels.register`` instead -- the two cannot both define it.
"""

import torch

from . import kernels, schemas, twins

lib = torch.library.Library("quantized_ops", "DEF")
for _schema in schemas.all_schemas().values():
    lib.define(_schema)
kernels.register(lib, fakes=True)
twins.register_layout_twins(lib)
