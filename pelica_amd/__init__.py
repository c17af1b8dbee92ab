"""pelica_amd — MI355X-native attention path for Pelica.

The compute lives in ``lib/libpelica_attn.so`` (HIP kernels for gfx950 behind
the C ABI declared in ``include/pelica_attn.h``).  ``pelica_amd.attn`` is the
host-side binding: it loads that library (failing loudly when it is missing)
and exposes the decode / prefill / partials-merge entry points on torch
device tensors.
"""
from .attn import (  # noqa: F401
    AttnDesc,
    AttnError,
    Shape,
    decode,
    library_path,
    load_library,
    new_workspace,
    partials_merge,
    prefill,
    prof_enable,
    prof_read,
    workspace_bytes,
)

__all__ = [
    "AttnDesc",
    "AttnError",
    "Shape",
    "decode",
    "library_path",
    "load_library",
    "new_workspace",
    "partials_merge",
    "prefill",
    "prof_enable",
    "prof_read",
    "workspace_bytes",
]
