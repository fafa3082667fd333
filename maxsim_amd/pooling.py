"""Token pooling for the pooled_binary corpus mode (reference: src/maxsim/pooling.py:1-57).

Each document of n tokens is reduced to ceil(n / factor) tokens: Ward
hierarchical clustering of the L2-normalised tokens (scipy), cut into at most
that many clusters, each replaced by the float64 mean of its original tokens.
Host-side index preparation; deterministic for a given input.
"""
from __future__ import annotations

import math

import numpy as np


def pool_doc_tokens(doc_embeddings: np.ndarray, doc_offsets: np.ndarray, factor: int):
    """(pooled embeddings f32 [T', dim], pooled offsets i64 [N + 1])."""
    if factor < 1:
        raise ValueError("factor must be >= 1")
    if factor == 1:
        return doc_embeddings.copy(), doc_offsets.copy()
    from scipy.cluster.hierarchy import fcluster, linkage

    chunks, offsets = [], [0]
    for start, end in zip(doc_offsets[:-1], doc_offsets[1:]):
        tokens = doc_embeddings[int(start):int(end)]
        n = tokens.shape[0]
        target = max(1, math.ceil(n / factor)) if n else 0
        if n == 0 or n <= target:
            if n:
                chunks.append(tokens.astype(np.float32, copy=True))
            offsets.append(offsets[-1] + n)
            continue
        unit = tokens / np.maximum(np.linalg.norm(tokens, axis=1, keepdims=True), 1e-12)
        labels = fcluster(linkage(unit, method="ward"), t=target, criterion="maxclust")
        clusters = int(labels.max())
        pooled = np.stack([tokens[labels == c].mean(axis=0, dtype=np.float64) for c in range(1, clusters + 1)])
        chunks.append(pooled.astype(np.float32))
        offsets.append(offsets[-1] + clusters)
    dim = doc_embeddings.shape[1]
    pooled_all = np.concatenate(chunks).astype(np.float32) if chunks else np.empty((0, dim), np.float32)
    return pooled_all, np.asarray(offsets, dtype=np.int64)
