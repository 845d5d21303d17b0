"""Cortex-Engine inference forward for AMD Instinct MI355X (gfx950).

Keeps the reference package layout (``cortex.kernels``, ``cortex.quantization``,
``cortex.models``); every op on a ROCm device runs on hand-written HIP kernels in
``libcortex_hip.so`` (see ``include/cortex_hip.h``).
"""

__version__ = "0.1.0"
