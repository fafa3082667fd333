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
from maxsim_amd.binres import BinaryResidualPackedDocs, binres_cascade_topk, binres_score, pack_binary_residual
from maxsim_amd.cascade import (
    ResidualInt4PackedDocs,
    cascade_topk,
    pack_residual_int4,
    prefix_score,
    prefix_topk,
    residual_int4_to_device,
    residual_score,
)
from maxsim_amd.experimental import (
    Int4PackedDocs,
    int4_maxsim,
    int4_maxsim_int8q,
    int4_to_device,
    pack_int4_symmetric,
    pack_int4_symmetric_device,
    topk_int4_maxsim,
)

from maxsim_amd.sdk import MODE_PRESETS, Corpus, CorpusMemoryReport, Index, Reranker, SearchResult

__all__ = [
    "BinaryResidualPackedDocs",
    "Corpus",
    "CorpusMemoryReport",
    "Index",
    "MODE_PRESETS",
    "Reranker",
    "ResidualInt4PackedDocs",
    "SearchResult",
    "binres_cascade_topk",
    "binres_score",
    "cascade_topk",
    "pack_binary_residual",
    "pack_residual_int4",
    "prefix_score",
    "prefix_topk",
    "residual_int4_to_device",
    "residual_score",
    "Int4PackedDocs",
    "PackedDocs",
    "int4_maxsim",
    "int4_maxsim_int8q",
    "int4_to_device",
    "maxsim",
    "pack_int4_symmetric",
    "pack_int4_symmetric_device",
    "pack_query_signs",
    "pack_signs",
    "score",
    "to_device",
    "topk_int4_maxsim",
    "topk_maxsim",
]
