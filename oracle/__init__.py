"""CPU oracle for the bitgpu attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain numpy (``oracle.ref``) and plain C (``oracle/pack_ref.c``),
the arithmetic of the reference's attention path (stfurkan/bitgpu v0.19.1). Every function
cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only as the checker (or the timed CPU baseline). The product path
(``bitgpu_amd``) never imports, links or calls anything here; it fails loudly when its HIP
library is missing.

Pinning status of each function is listed in ``oracle/ref.py``'s module docstring.
"""
