"""Brute-force retrieval scoring over dense vectors on the device: the host
side of topRetrievalScores / dotRetrievalVectors
(runtime/retrieval_eval.go:586-661).

`DenseRetrievalIndex` binds the document vectors once, in ascending doc-ID
order, so that the device top-k's (score desc, row asc) order is
retrievalScoreBetter's (score desc, doc ID asc; Go compares strings
bytewise, which for UTF-8 is code-point order, Python's).  Two docs with the
same ID keep their input order.  `top` returns, per query, the
(doc ID, score) pairs topRetrievalScores returns, scores bit-identical to
the reference's f32 loop.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np

from .rocm import DeviceArray, Runtime


class DenseRetrievalIndex:
    def __init__(self, rt: Runtime, vectors: np.ndarray, ids: Sequence[str], f16: bool = False):
        """vectors: [n, d] f32 values (f16=True stores them as binary16,
        which is exact only for values f16 represents; the scores are then
        those of the f16-representable values)."""
        vectors = np.asarray(vectors, np.float32)
        if vectors.ndim != 2 or vectors.shape[0] != len(ids):
            raise ValueError("vectors [n, d] and n ids expected")
        self.rt = rt
        self.order = np.array(sorted(range(len(ids)), key=lambda i: (ids[i], i)), dtype=np.int64)
        self.ids = [ids[i] for i in self.order]
        rows = np.ascontiguousarray(vectors[self.order])
        if f16:
            rows16 = rows.astype(np.float16)
            if not np.array_equal(rows16.astype(np.float32), rows):
                raise ValueError("f16 storage would round these vectors; keep them in f32")
            rows = rows16.view(np.uint16)
        self.rows = rt.to_device(rows)
        self.n, self.d = vectors.shape

    def scores(self, queries: np.ndarray) -> np.ndarray:
        """dotRetrievalVectors of each query against every doc, in the
        caller's doc order: f32 [nq, n]."""
        q = np.ascontiguousarray(np.atleast_2d(np.asarray(queries, np.float32)))
        s = self.rt.dense_scores(self.rows, self.rt.to_device(q)).download()
        out = np.empty_like(s)
        out[:, self.order] = s
        return out

    def top(self, queries: np.ndarray, top_k: int) -> List[List[Tuple[str, float]]]:
        """topRetrievalScores for each query (top_k <= 0 or > n: every doc)."""
        q = np.ascontiguousarray(np.atleast_2d(np.asarray(queries, np.float32)))
        k = self.n if top_k <= 0 or top_k > self.n else top_k
        ids, scores = self.rt.dense_topk(self.rows, self.rt.to_device(q), k)
        ids, scores = ids.download(), scores.download()
        return [[(self.ids[int(r)], float(s)) for r, s in zip(ids[i], scores[i])] for i in range(q.shape[0])]
