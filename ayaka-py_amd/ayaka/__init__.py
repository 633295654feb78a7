"""MI355X-native (gfx950) FP8 linear path with Ayaka's layer, recipe and operator API.

Public entry points mirror the reference package layout:

* ``ayaka.layers.linear.fp8`` -- the FP8 ``LinearMethod`` classes and ``FP8Config``;
* ``ayaka.model_loader.fp8`` -- checkpoint recipe detection and scale contracts;
* ``ayaka.kernel.hip`` -- the ``torch.ops.ayaka.*`` operators, served by
  hand-written HIP kernels in ``libayaka_fp8.so`` through a C ABI.
"""

__version__ = "0.1.0"
