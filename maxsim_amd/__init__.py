"""maxsim_amd -- MI355X-native MaxSim scoring engine (HIP/gfx950).

Public names mirror the reference package ``maxsim`` (src/maxsim/__init__.py:1-36)
for the compressed scoring path: ``import maxsim_amd as maxsim``.
"""
from maxsim_amd._api import (
    PackedDocs,
    maxsim,
    pack_query_signs,
    pack_signs,
    score,
    to_device,
    topk_maxsim,
)
from maxsim_amd.experimental import (
    Int4PackedDocs,
    int4_maxsim,
    int4_maxsim_int8q,
    int4_to_device,
    pack_int4_symmetric,
    topk_int4_maxsim,
)

__all__ = [
    "Int4PackedDocs",
    "PackedDocs",
    "int4_maxsim",
    "int4_maxsim_int8q",
    "int4_to_device",
    "maxsim",
    "pack_int4_symmetric",
    "pack_query_signs",
    "pack_signs",
    "score",
    "to_device",
    "topk_int4_maxsim",
    "topk_maxsim",
]
