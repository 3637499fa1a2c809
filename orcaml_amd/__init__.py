"""MI355X (gfx950) backend for Orca's MLP training-step hot path.

liborca_hip.so (built by ``python -m orcaml_amd.build``) implements the
reference's ``Backend`` trait ops (orca-tensor/src/backend.rs:19-315) and the
fused training-step kernels behind the C ABI in include/orca_hip.h.  This
package is its Python binding:

* ``device``   -- HIP context, caching allocator, buffers, kernel timing;
* ``backend``  -- ``HipBackend``, the trait's methods over the C ABI;
* ``autodiff`` -- the reference tape and frontend op sequence replayed on a
                  backend (the unchanged composed path);
* ``mlp``      -- the device-resident fused MLP training step;
* ``synth``    -- seeded synthetic inputs.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
