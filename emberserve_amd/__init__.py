"""emberserve_amd: emberserve's fused per-layer elementwise ops as gfx950 (MI355X) HIP
kernels behind the reference's Python call signatures.

`emberserve_amd.ops` is the drop-in for `emberserve.model.ops`; `emberserve_amd.rope`
for `emberserve.model.rope`; `emberserve_amd.layers` holds the module-level drop-ins.
The kernels live in libember_ops.so (C ABI: include/ember_ops.h), built by
`python -m emberserve_amd.build`.
"""

from . import ops, rope, layers  # noqa: F401

__all__ = ["ops", "rope", "layers"]
