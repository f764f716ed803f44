"""DSA lightning-indexer selection on the CPU (test infrastructure only).

Restates DSAState.update_and_select (runtime/glm_dsa.py:113-166) from the
point where the index queries, keys and head weights exist:
  scores[s] = sum_j w_head[j] * max((q_idx[j] . k_idx[s]) * head_dim^-0.5, 0)
                                                          fp32   (:147-150)
  keys s > query position are excluded (causal)                  (:152-155)
  the index_topk highest scores, indices in ascending order      (:156-160)
and the gather that feeds absorbed MLA (runtime/glm.py:285-289).  Where
several keys tie at the k-th score, the lowest indices are kept (argpartition
leaves that choice open).
"""

from __future__ import annotations

import numpy as np


def index_scores(q_idx: np.ndarray, w_head: np.ndarray, k_idx: np.ndarray,
                 scale: float) -> np.ndarray:
    """q_idx [NH, D], w_head [NH], k_idx [S, D] -> scores [S] fp32."""
    q = q_idx.astype(np.float32)
    k = k_idx.astype(np.float32)
    s = (q @ k.T) * np.float32(scale)                       # [NH, S]
    s = np.maximum(s, np.float32(0.0))
    return (s * w_head.astype(np.float32)[:, None]).sum(axis=0, dtype=np.float32)


def topk(scores: np.ndarray, n: int, k: int) -> np.ndarray:
    """Ascending indices of the k highest of scores[:n] (all of them if n <= k);
    ties at the k-th score keep the lowest indices."""
    n = min(int(n), scores.shape[0])
    if n <= k:
        return np.arange(n, dtype=np.int64)
    idx = np.arange(n)
    order = np.lexsort((idx, -scores[:n].astype(np.float64)))
    return np.sort(order[:k])


def select(q_idx: np.ndarray, w_head: np.ndarray, k_idx: np.ndarray, n: int, k: int,
           scale: float) -> np.ndarray:
    """Selection of one decode query over the first n cached keys."""
    return topk(index_scores(q_idx, w_head, k_idx[:n], scale), n, k)


def gather(latent: np.ndarray, sel: np.ndarray) -> np.ndarray:
    """The selected latent rows, in selection order (runtime/glm.py:288)."""
    return latent[sel]


def select_torch(q_idx, w_head, k_idx, k: int, scale: float):
    """Scores and top-k of one decode query in torch on the CPU (the timed CPU
    baseline): q_idx [NH, D], w_head [NH], k_idx [S, D] -> ascending indices
    of the k highest scores (torch.topk; ties in unspecified order)."""
    import torch

    s = torch.relu((q_idx.float() @ k_idx.float().T) * scale)          # [NH, S]
    scores = (s * w_head.float()[:, None]).sum(dim=0)
    if scores.numel() <= k:
        return torch.arange(scores.numel())
    return torch.sort(torch.topk(scores, k).indices).values
