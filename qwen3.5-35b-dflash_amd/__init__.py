"""MI355X-native (gfx950) W4A16 qlinear and routed-MoE expert FFN.

The directory name is not a Python identifier; load it under the alias
``qwen35_dflash_amd`` (see ``load_package`` in ``tests/conftest.py`` and
``bench.py``).  Modules:

* ``fused_ops`` -- FusedOps ABI-v1 adapter module (the drop-in seam)
* ``ops``       -- PyTorch-ROCm wrappers over the C ABI
* ``packing``   -- ``PackedW4`` / ``SharedExpert`` types and the int4 packer
* ``plan``      -- tensor inventory of the target (names, shapes, which are int4)
* ``layers``    -- non-hot decoder arithmetic (delta rule, norms, rotary, attention)
* ``target``    -- the verify forward of the whole target on the HIP kernels
* ``quantized`` -- the quantized-weights seam (``OriginalQuantizedWeights`` interface)
* ``checkpoint`` -- readers of the original safetensors shards and the portable weight cache
* ``session``   -- target session with a batched speculative verify
* ``synthetic`` -- seeded synthetic workloads (tests and benchmark)
* ``_lib``      -- ctypes binding of ``libdflash_hip.so``
* ``build``     -- hipcc build recipe
"""
from . import _lib, checkpoint, fused_ops, layers, ops, packing, plan, quantized, session, synthetic, target  # noqa: F401
from .packing import PackedW4, SharedExpert, concat_rows, pack_int4, quantize_w4  # noqa: F401
