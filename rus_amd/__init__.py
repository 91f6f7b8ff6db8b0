"""rus_amd — MI355X (gfx950) implementation of the fused QLoRA training hot path of
fokyso82002-rgb/rus (its ``solution/`` package).

Modules mirror the reference's layout so they can be used as a drop-in:

* ``rus_amd.kernels``  — launchers with the reference's names (kernels.py), backed by hand-written
  HIP kernels in ``librus_amd.so`` through the C ABI of ``include/rus_amd.h``;
* ``rus_amd.quant``    — NF4 double-quant quantisation (model-load step).
"""

from __future__ import annotations

__version__ = "0.1.0"
