"""Seeded synthetic multi-vector corpora for the benchmark configurations.

Generator (the reference has none; this fixes one):
  * seed default 20260713 (the reference's canonical seed, run_cuda_step1.py:101);
  * document lengths ``rng.integers(lo, hi + 1)``, uniform inclusive;
  * documents are generated in blocks of ``BLOCK_DOCS`` documents, each block
    from its own child generator (``SeedSequence(seed).spawn``), so a corpus of
    any size is produced with bounded memory and reproducibly;
  * per document a centroid c ~ N(0, I_dim); tokens = c + eps, eps ~ N(0, 0.5^2)
    i.i.d. per coordinate (sigma = 0.5); every token L2-normalised (float32);
  * query b: a seeded source document; 32 of its tokens (without replacement
    when it has at least 32, else with replacement) plus N(0, 0.1^2) noise
    (sigma = 0.1), L2-normalised per token.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SEED = 20260713
BLOCK_DOCS = 1024
TOKEN_SIGMA = 0.5
QUERY_SIGMA = 0.1


@dataclass(frozen=True)
class Corpus:
    embeddings: np.ndarray  # f32 [T, dim]
    offsets: np.ndarray  # i64 [N + 1]
    lengths: np.ndarray  # i64 [N]


def _normalize(x: np.ndarray) -> np.ndarray:
    norms = np.linalg.norm(x, axis=1, keepdims=True)
    norms[norms == 0] = 1.0
    return (x / norms).astype(np.float32, copy=False)


def doc_lengths(num_docs: int, lo: int, hi: int, seed: int = SEED) -> np.ndarray:
    rng = np.random.default_rng(np.random.SeedSequence(seed).spawn(1)[0])
    return rng.integers(lo, hi + 1, size=num_docs).astype(np.int64)


def iter_blocks(num_docs: int, lo: int, hi: int, dim: int = 128, seed: int = SEED):
    """Yield (first_doc, lengths, embeddings f32) per block of BLOCK_DOCS docs."""
    lengths = doc_lengths(num_docs, lo, hi, seed)
    children = np.random.SeedSequence(seed).spawn(2 + (num_docs + BLOCK_DOCS - 1) // BLOCK_DOCS)[2:]
    for block, child in enumerate(children):
        first = block * BLOCK_DOCS
        lens = lengths[first : first + BLOCK_DOCS]
        rng = np.random.default_rng(child)
        centroids = rng.standard_normal((lens.shape[0], dim), dtype=np.float32)
        tokens = np.repeat(centroids, lens, axis=0)
        tokens += rng.standard_normal(tokens.shape, dtype=np.float32) * np.float32(TOKEN_SIGMA)
        yield first, lens, _normalize(tokens)


def make_corpus(num_docs: int, lo: int, hi: int, dim: int = 128, seed: int = SEED) -> Corpus:
    lengths = doc_lengths(num_docs, lo, hi, seed)
    offsets = np.zeros(num_docs + 1, np.int64)
    np.cumsum(lengths, out=offsets[1:])
    emb = np.empty((int(offsets[-1]), dim), np.float32)
    for first, lens, block in iter_blocks(num_docs, lo, hi, dim, seed):
        start = int(offsets[first])
        emb[start : start + block.shape[0]] = block
    return Corpus(emb, offsets, lengths)


def make_queries(corpus: Corpus, batch: int, query_tokens: int = 32, seed: int = SEED) -> np.ndarray:
    """f32 [batch, query_tokens, dim] built from perturbed tokens of seeded docs."""
    rng = np.random.default_rng(np.random.SeedSequence(seed).spawn(2)[1])
    dim = corpus.embeddings.shape[1]
    num_docs = corpus.offsets.shape[0] - 1
    out = np.empty((batch, query_tokens, dim), np.float32)
    for b in range(batch):
        doc = int(rng.integers(0, num_docs))
        while corpus.lengths[doc] == 0:
            doc = int(rng.integers(0, num_docs))
        start, length = int(corpus.offsets[doc]), int(corpus.lengths[doc])
        pick = rng.choice(length, size=query_tokens, replace=length < query_tokens)
        q = corpus.embeddings[start + pick] + rng.standard_normal((query_tokens, dim), dtype=np.float32) * np.float32(QUERY_SIGMA)
        out[b] = _normalize(q)
    return out


def query_weights(batch: int, query_tokens: int, seed: int = SEED) -> np.ndarray:
    """Per-(batch, query token) weights uniform in [0.5, 1.5] (config 3)."""
    rng = np.random.default_rng(np.random.SeedSequence(seed + 1).spawn(1)[0])
    return rng.uniform(0.5, 1.5, size=(batch, query_tokens)).astype(np.float32)


# The BASELINE.json configurations (lo, hi tokens per document, num_docs).
CONFIGS = {
    1: dict(num_docs=512, lo=32, hi=64, batch=1),
    2: dict(num_docs=4096, lo=64, hi=192, batch=4),
    3: dict(num_docs=4096, lo=64, hi=192, batch=4),
    4: dict(num_docs=10240, lo=256, hi=1024, batch=256),
    5: dict(num_docs=4096, lo=64, hi=192, batch=4),
}
