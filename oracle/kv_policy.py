"""PagedKVCache bookkeeping restated shape-free (test infrastructure only).

Follows runtime/kv_paged.py:
  update (:143-162)  tokens join the layer's tail; full pages close; after the
                     last layer the offset advances and the budget is enforced
  nbytes (:187-194)  resident closed pages + tail tokens
  _enforce_budget (:216-240)  spill oldest page index first, round-robin over
                     layers, skipping the newest `resident_pages` closed pages
                     of each layer and pages already spilled; stop as soon as
                     nbytes() <= max_bytes
Bytes are counted per token (token_bytes = K+V bytes of one position across
the batch and heads), so a closed page costs page_positions * token_bytes.
"""

from __future__ import annotations


class PagedKVPolicy:
    def __init__(self, num_layers: int, max_bytes: int, page_positions: int,
                 resident_pages: int, token_bytes: int):
        self.num_layers = num_layers
        self.max_bytes = max_bytes
        self.page_positions = page_positions
        self.resident_pages = resident_pages
        self.token_bytes = token_bytes
        self.pages = [[] for _ in range(num_layers)]   # list of resident flags
        self.tail = [0] * num_layers
        self.offset = 0
        self.spill_log: list[tuple[int, int]] = []

    def nbytes(self) -> int:
        page = self.page_positions * self.token_bytes
        return sum(sum(page for r in p if r) + t * self.token_bytes
                   for p, t in zip(self.pages, self.tail))

    def update(self, layer: int, n_tokens: int) -> list[tuple[int, int]]:
        self.tail[layer] += n_tokens
        while self.tail[layer] >= self.page_positions:
            self.pages[layer].append(True)
            self.tail[layer] -= self.page_positions
        spilled = []
        if layer == self.num_layers - 1:
            self.offset += n_tokens
            spilled = self._enforce_budget()
        return spilled

    def _enforce_budget(self) -> list[tuple[int, int]]:
        out = []
        if self.nbytes() <= self.max_bytes:
            return out
        for page_idx in range(max(len(p) for p in self.pages)):
            for layer in range(self.num_layers):
                pages = self.pages[layer]
                if page_idx >= len(pages) - self.resident_pages:
                    continue
                if not pages[page_idx]:
                    continue
                pages[page_idx] = False
                out.append((layer, page_idx))
                self.spill_log.append((layer, page_idx))
                if self.nbytes() <= self.max_bytes:
                    return out
        return out
