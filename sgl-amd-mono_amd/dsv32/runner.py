"""Host runner of the DSA layer launches: build key, step tables, caches.

Mirrors the reference's runner structs (``sgl_amd_mono/glm53/gfx950/runner.py:32-111``)
and the per-step row tables its spec builds (``sgl_amd_mono/glm53/spec.py:467-496``):

* ``Dsv32Build``: what a compiled launch is specialised on (width, TP size, launches per
  step, indexer or not, the indexer's key bound, weight layout, KV dtype, the test
  fault injection).
* ``Dsv32Step``: the rows of one decode or verify step, shared by every layer's launch:
  positions (clamped into the served context), KV slots (-1 for a pad row), ``indptr``
  (row s attends ``min(position + 1, 2048)`` keys), request ids, the page table and the
  compact top-k buffer (row s at ``indptr[s]``; the last entry takes the copies of a
  row's unused keys).
* ``Dsv32Caches``: a layer's MLA KV cache and index-key cache, bound in place.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .config import DSV32

TOPK = DSV32.index_topk  # keys a row attends at most (the indexer's top-k)


@dataclass(frozen=True)
class Dsv32Build:
    rows: int
    tp: int = 4
    launches_per_step: int = 1
    with_indexer: bool = True
    index_max_seq: int = 0
    layout: str = "aiter16"
    kv_fp8: bool = True
    fault_site: int = 0
    fault_after: int = 0


@dataclass
class Dsv32Step:
    positions: torch.Tensor  # i64 [W]
    slots: torch.Tensor  # i64 [W], -1 for a pad row
    indptr: torch.Tensor  # i32 [W + 1]
    req_ids: torch.Tensor  # i32 [W]
    page_table: torch.Tensor  # i32 [requests, pages]
    topk: torch.Tensor  # i32 [W * TOPK + 1]


@dataclass
class Dsv32Caches:
    kv: torch.Tensor  # [slots, kv_row] E4M3 (or bf16)
    idx: Optional[torch.Tensor] = None  # index-key pages, uint8


def alloc_step(width: int, device) -> Dsv32Step:
    """The step tables of a width, allocated once (rewritten every step, in the graph
    when captured)."""
    i32, i64 = torch.int32, torch.int64
    return Dsv32Step(
        positions=torch.zeros(width, dtype=i64, device=device),
        slots=torch.full((width,), -1, dtype=i64, device=device),
        indptr=torch.zeros(width + 1, dtype=i32, device=device),
        req_ids=torch.zeros(width, dtype=i32, device=device),
        page_table=torch.zeros(width, 1, dtype=i32, device=device),
        topk=torch.zeros(width * TOPK + 1, dtype=i32, device=device),
    )


def fill_step(st: Dsv32Step, positions: torch.Tensor, out_cache_loc: torch.Tensor, rows: int,
              max_position: int, page_table: Optional[torch.Tensor] = None) -> Dsv32Step:
    """Write the rows of a step into ``st`` in place (``glm53/spec.py:467-496``).

    SGLang's slot 0 is its padding slot: such a row writes no cache and attends no key.
    Verify rows past the context keep their position inside the rotary table and the
    indexer's score rows. A row sees keys 0 ..= its position, at most TOPK of them (in a
    verify step ``seq_lens`` holds each request's prefix, not each row's keys, so the
    count comes from the position)."""
    S, W = rows, st.positions.shape[0]
    if not 0 < S <= W:
        raise ValueError(f"a step of {S} rows at width {W}")
    loc = out_cache_loc[:S].to(torch.int64)
    valid = loc != 0
    st.slots[:S] = torch.where(valid, loc, torch.full_like(loc, -1))
    st.slots[S:] = -1
    pos = positions[:S].to(torch.int64).clamp(max=max_position)
    st.positions[:S] = pos
    st.positions[S:] = 0
    count = torch.where(valid, (pos + 1).clamp(max=TOPK), torch.zeros_like(pos))
    st.indptr[0] = 0
    st.indptr[1 : S + 1] = torch.cumsum(count, 0).to(torch.int32)
    st.indptr[S + 1 :] = st.indptr[S]
    st.req_ids[:S] = torch.arange(S, dtype=torch.int32, device=loc.device)
    st.req_ids[S:] = 0
    if page_table is not None:
        st.page_table = page_table[:S]
    return st


def take_topk(st: Dsv32Step, topk_indices: torch.Tensor, rows: int) -> None:
    """A previous layer's top-k (SGLang's [S, TOPK] KV slots, -1 past a row's keys) into
    the compact buffer a launch reads, row s at ``indptr[s]``; entries past a row's
    count go to the last (spare) entry (``glm53/spec.py:419-429``)."""
    S = rows
    W = st.positions.shape[0]
    cols = torch.arange(TOPK, dtype=torch.int64, device=st.topk.device)
    start = st.indptr[:S].to(torch.int64).unsqueeze(1)
    count = (st.indptr[1 : S + 1] - st.indptr[:S]).to(torch.int64).unsqueeze(1)
    dst = torch.where(cols < count, start + cols, torch.full_like(cols, W * TOPK))
    st.topk.scatter_(0, dst.reshape(-1), topk_indices[:S].reshape(-1).to(torch.int32))


def page_table(req_to_token: torch.Tensor, req_pool_indices: torch.Tensor, rows: int,
               context: int, page: int = DSV32.page) -> torch.Tensor:
    """The rows' page tables i32 [rows, pages] from SGLang's ``req_to_token`` (a request's
    KV slot at every position; pages of ``page`` slots): a page id is the slot of the
    page's first position divided by ``page``. Row s is request s of the step (the
    launches' request ids)."""
    pages = -(-context // page)
    first = req_to_token[req_pool_indices[:rows].to(torch.int64)][:, : pages * page : page]
    return (first.to(torch.int64) // page).to(torch.int32).contiguous()
