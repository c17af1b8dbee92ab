"""pelica_amd — MI355X-native attention path for Pelica.

The compute lives in ``lib/libpelica_attn.so`` (HIP kernels for gfx950 behind
the C ABI declared in ``include/pelica_attn.h``).  ``pelica_amd.attn`` is the
host-side binding: it loads that library (failing loudly when it is missing)
and exposes every entry point on torch device tensors.
"""
from .attn import (  # noqa: F401
    AttnDesc,
    AttnError,
    Rope,
    Shape,
    decode,
    decode_noalloc,
    decode_partials,
    decode_partials_range,
    default_scale,
    library_path,
    load_library,
    make_desc,
    mla,
    new_workspace,
    partials_merge,
    partials_merge_batch,
    prefill,
    prefill_round,
    prof_enable,
    prof_read,
    qkv_rope_cache,
    reload_tuning,
    token_stride,
    workspace_bytes,
)

__all__ = [
    "AttnDesc",
    "AttnError",
    "Rope",
    "Shape",
    "decode",
    "decode_noalloc",
    "decode_partials",
    "decode_partials_range",
    "default_scale",
    "library_path",
    "load_library",
    "make_desc",
    "mla",
    "new_workspace",
    "partials_merge",
    "partials_merge_batch",
    "prefill",
    "prefill_round",
    "prof_enable",
    "prof_read",
    "qkv_rope_cache",
    "reload_tuning",
    "token_stride",
    "workspace_bytes",
]
