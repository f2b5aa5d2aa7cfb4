"""MI355X (gfx950) DSA sparse-attention hot path for GLM-5.1 / DeepSeek-V3.2.

Hand-written HIP kernels behind a C ABI (include/mi355_dsa.h,
libmi355_dsa.so), registered as torch custom ops with the reference's
schemas and wrapped by a _sm70_ops-compatible module.

The directory name contains dashes, so it is imported through a loader that
registers it as the module `glm5_on_v100_amd` (see __graft_entry__.py or
tests/conftest.py).
"""
from . import _lib, ops, _sm70_ops, _cache_ops, dsa_layer, mla_prefill, synthetic  # noqa: F401

__all__ = ["_lib", "ops", "_sm70_ops", "_cache_ops", "dsa_layer", "mla_prefill", "synthetic",
           "load_library"]


def load_library():
    """Loads libmi355_dsa.so (raising if it is not built) and registers ops."""
    L = _lib.lib()
    ops.register()
    return L
