"""Per-step row tables of the DSA layer launches.

A decode step of ``rows`` rows runs at a built width W >= rows; every covered layer of the
step reads the same tables, so they are written once a step (inside the captured graph
when SGLang replays one). The rules are the reference's step contract
(``sgl_amd_mono/glm53/spec.py:467-496``, pinned by its unit cases
``test/unit/test_glm53_spec.py:127-158``, transcribed in ``tests/golden/step_tables.json``):

* a row whose ``out_cache_loc`` is 0 is padding (SGLang's slot 0): it writes no cache
  (slot -1) and attends no key;
* a position past the served context is clamped to its last position (the rotary table
  and the indexer's score rows end there);
* a live row attends ``min(position + 1, 2048)`` keys; ``indptr()`` is the running sum of
  those counts, constant past the last row. No launch reads it (each launch takes the
  positions and slots and ranks a row's keys itself), so it is derived on demand and not
  rewritten inside a captured step;
* row s is request s of the step (decode: one row a request).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .config import DSV32

TOPK = DSV32.index_topk  # keys a row attends at most (the indexer's top-k)


@dataclass
class StepRows:
    """The tables of one width W: positions i64 [W], cache slots i64 [W] (-1: no write),
    request ids i32 [W] and the page table i32 [requests, pages] (a view of SGLang's, or
    of ``pages``, the table's own full-width buffer, set by ``write``)."""

    positions: torch.Tensor
    slots: torch.Tensor
    req_ids: torch.Tensor
    page_table: torch.Tensor
    pages: Optional[torch.Tensor] = None

    @classmethod
    def empty(cls, width: int, device, context: int = 0) -> "StepRows":
        """Tables of ``width`` rows, all padding, allocated once and rewritten each step;
        with ``context`` > 0 also a page-table buffer wide enough for that many keys."""
        kw = dict(device=device)
        npages = -(-context // DSV32.page)
        pages = torch.zeros(width, npages, dtype=torch.int32, **kw) if npages else None
        return cls(positions=torch.zeros(width, dtype=torch.int64, **kw),
                   slots=torch.full((width,), -1, dtype=torch.int64, **kw),
                   req_ids=torch.zeros(width, dtype=torch.int32, **kw),
                   page_table=torch.zeros(width, 1, dtype=torch.int32, **kw), pages=pages)

    @property
    def width(self) -> int:
        return self.positions.numel()

    def write(self, positions: torch.Tensor, out_cache_loc: torch.Tensor, rows: int,
              max_position: int, page_table: Optional[torch.Tensor] = None) -> "StepRows":
        """Rewrite the tables in place for a step of ``rows`` rows (with tensor ops only,
        so the writes are captured with the step). Returns self."""
        W = self.width
        if rows < 1 or rows > W:
            raise ValueError(f"a step of {rows} rows does not fit width {W}")
        loc = out_cache_loc[:rows].to(torch.int64)
        pad = loc == 0
        self.slots.fill_(-1)
        self.slots[:rows].copy_(loc.masked_fill(pad, -1))
        pos = positions[:rows].to(torch.int64).clamp(max=max_position)
        self.positions.zero_()
        self.positions[:rows].copy_(pos)
        self.req_ids.zero_()
        self.req_ids[:rows].copy_(torch.arange(rows, dtype=torch.int32, device=loc.device))
        if page_table is not None:
            self.page_table = page_table[:rows]
        return self

    def fill_pages(self, req_to_token: torch.Tensor, req_pool_indices: torch.Tensor,
                   rows: int) -> torch.Tensor:
        """Write the first ``rows`` rows of the ``pages`` buffer from SGLang's
        ``req_to_token`` (``page_table``'s rule; pages past the pool's width hold 0) and
        return that view."""
        if self.pages is None:
            raise ValueError("StepRows built without a page-table buffer (context 0)")
        npages = self.pages.shape[1]
        page = DSV32.page
        have = min(npages, -(-req_to_token.shape[1] // page))
        first = req_to_token.index_select(0, req_pool_indices[:rows].to(torch.int64))
        view = self.pages[:rows]
        view[:, :have].copy_(first[:, : have * page : page].to(torch.int64) // page)
        if have < npages:
            view[:, have:].zero_()
        return view

    def indptr(self) -> torch.Tensor:
        """i32 [W + 1]: row s attends keys indptr[s] .. indptr[s + 1] (pad rows none)."""
        keys = (self.positions + 1).clamp(max=TOPK).masked_fill(self.slots < 0, 0)
        out = torch.zeros(self.width + 1, dtype=torch.int32, device=self.positions.device)
        out[1:] = torch.cumsum(keys, 0).to(torch.int32)
        return out

    def rows(self, n: int):
        """The first n rows' positions, slots and request ids (the launches' [R] tables)."""
        return self.positions[:n], self.slots[:n], self.req_ids[:n]


def page_table(req_to_token: torch.Tensor, req_pool_indices: torch.Tensor, rows: int,
               context: int, page: int = DSV32.page) -> torch.Tensor:
    """Page ids i32 [rows, pages] from SGLang's ``req_to_token`` (each request's KV slot at
    every position, pages of ``page`` consecutive slots): a page's id is the slot of its
    first position over ``page``. For a backend whose metadata carries no page table."""
    pages = -(-context // page)
    first = req_to_token[req_pool_indices[:rows].to(torch.int64)][:, : pages * page : page]
    return (first.to(torch.int64) // page).to(torch.int32).contiguous()
