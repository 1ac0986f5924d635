"""Training items and the concatenated (unpadded) batch layout.

``TrainingItem`` mirrors the reference record (src/StructuredDecisions.Laya.Training/TrainableDecisionModel.cs:11-28).
``Batch`` is what ``Forward`` builds before any math (TrainableDecisionModel.cs:254-274): items
concatenated with no padding, one segment per item, marker rows ``segment.Start + max(0, marker)``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import numpy as np


@dataclass
class TrainingItem:
    token_ids: np.ndarray
    marker_positions: np.ndarray
    question_type: int
    target: np.ndarray

    @property
    def options(self) -> int:
        return len(self.marker_positions)

    @property
    def label(self) -> int:
        return int(np.argmax(self.target)) if len(self.target) else 0


@dataclass
class Batch:
    lengths: np.ndarray      # int32 [items]
    tokens: np.ndarray       # int32 [Σ lengths]
    n_options: np.ndarray    # int32 [items]
    markers: np.ndarray      # int32 [Σ options], positions inside each item
    qtypes: np.ndarray       # int32 [items]

    @classmethod
    def from_items(cls, items: Sequence[TrainingItem]) -> "Batch":
        return cls(
            lengths=np.array([len(i.token_ids) for i in items], dtype=np.int32),
            tokens=np.concatenate([np.asarray(i.token_ids, dtype=np.int32) for i in items]) if items
            else np.zeros(0, np.int32),
            n_options=np.array([i.options for i in items], dtype=np.int32),
            markers=np.concatenate([np.asarray(i.marker_positions, dtype=np.int32) for i in items]) if items
            else np.zeros(0, np.int32),
            qtypes=np.array([i.question_type for i in items], dtype=np.int32),
        )

    @property
    def n_items(self) -> int:
        return len(self.lengths)

    @property
    def n_tokens(self) -> int:
        return int(self.lengths.sum())

    @property
    def n_markers(self) -> int:
        return int(self.n_options.sum())

    def starts(self) -> np.ndarray:
        return (np.concatenate([[0], np.cumsum(self.lengths)[:-1]]) if len(self.lengths) else
                np.zeros(0)).astype(np.int32)

    def marker_rows(self) -> np.ndarray:
        starts = np.repeat(self.starts(), self.n_options)
        return (starts + np.maximum(self.markers, 0)).astype(np.int32)

    def split(self, per_option: np.ndarray) -> List[np.ndarray]:
        out, o = [], 0
        for k in self.n_options:
            out.append(np.asarray(per_option[o:o + k]))
            o += int(k)
        return out


def synthetic_batch(rng: np.random.Generator, lengths: Sequence[int], n_options: Sequence[int],
                    qtypes: Sequence[int], vocab: int, zipf: float = 0.0) -> Batch:
    """Random ids (uniform, or Zipf(s) ranks mapped to ids rank-1) with markers at 1 + 2k."""
    lengths = [int(x) for x in lengths]
    total = sum(lengths)
    if zipf > 0:
        ranks = np.arange(1, vocab + 1, dtype=np.float64)
        p = ranks ** (-zipf)
        p /= p.sum()
        tokens = rng.choice(vocab, size=total, p=p).astype(np.int32)
    else:
        tokens = rng.integers(0, vocab, size=total, dtype=np.int64).astype(np.int32)
    markers = []
    for L, k in zip(lengths, n_options):
        markers.extend(min(1 + 2 * j, L - 1) for j in range(k))
    return Batch(lengths=np.array(lengths, np.int32), tokens=tokens, n_options=np.array(n_options, np.int32),
                 markers=np.array(markers, np.int32), qtypes=np.array(qtypes, np.int32))
