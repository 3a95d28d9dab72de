"""Slot and page bookkeeping for the paged KV cache, and the block table the kernels read.

Drop-in for reference `src/torch_llm/inference/page_allocator.py:9-366`. The public
names, the argument meaning, the exception types and the order in which pages and
slots are handed out are the reference's (callers and tests depend on them); the
bookkeeping is organised around one lease record per occupied slot.

Host state (authoritative; nothing here is ever read back from the GPU):
  * `_leases[slot]`: the owning request, its pages in logical order and its
    committed token count, or None for a free slot;
  * `free_blocks`, `free_slots`: stacks. The next page or slot handed out is the
    last element, and released ones are pushed back on the end;
  * `request_to_slot`: request id -> slot.
Device state (what the kernels index):
  * `block_table [max_cache_slots, ceil(max_seq_len / block_size)]` int32: row s
    lists slot s's pages in logical order, -1 after them;
  * `seq_lens [max_cache_slots]` int32: committed lengths.

Every mutation checks the whole request first and only then changes state, so a
refused call (ValueError, CacheCapacityError) leaves the allocator as it was.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field

import torch as t

from aiproj_amd.inference.paged_kv_cache import PagedKVCache


class CacheCapacityError(RuntimeError):
    """Too few free pages or slots for an otherwise valid request."""


def _is_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def initialize_cache(kvcache_config, model_config, device):
    """The allocator shared by all layers, plus one PagedKVCache per layer
    (reference `page_allocator.py:13-36`)."""
    c = kvcache_config
    allocator = PageAllocator(c.num_blocks, c.block_size, c.max_cache_slots, c.cache_max_seq_len, device)
    storage = [
        PagedKVCache(c.num_blocks, c.block_size, model_config.num_kv_heads, model_config.head_dim, device,
                     cache_dtype=c.kv_cache_dtype, scale_dtype=c.kv_scale_dtype)
        for _ in range(model_config.num_layers)
    ]
    return allocator, storage


@dataclass
class CacheContainer:
    """What one batch's forward needs from the cache (reference `page_allocator.py:358-366`).

    `block_table` is the allocator's whole table: the decode kernel picks the row of
    sequence b as `block_table[cache_slots[b]]`. `physical_blocks`/`block_offsets`
    are the write locations of the batch's tokens, `context_lengths` the tokens each
    sequence attends over once the batch is written.

    `appends_last_position` (not in the reference; default False) is True only when
    the batch has one token per sequence and each token's write location is its
    sequence's last attended position, `context_lengths[b] - 1`. It lets the decode
    step write the new token inside the decode kernel; with False the step makes the
    append and the decode as two calls.
    """

    cache_slots: t.Tensor
    physical_blocks: t.Tensor
    block_offsets: t.Tensor
    context_lengths: t.Tensor
    block_table: t.Tensor
    appends_last_position: bool = False


@dataclass
class _Lease:
    request_id: int
    pages: list[int] = field(default_factory=list)
    committed: int = 0


class PageAllocator:
    """Owns slots and pages on the host; mirrors the kernel metadata on the device.

    One thread and one stream own an allocator; it takes no locks."""

    def __init__(self, num_blocks, block_size, max_cache_slots, max_seq_len, device):
        sizes = {"num_blocks": num_blocks, "block_size": block_size,
                 "max_cache_slots": max_cache_slots, "max_seq_len": max_seq_len}
        for name, value in sizes.items():
            if not _is_int(value) or value <= 0:
                raise ValueError(f"{name} must be a positive integer, got {value!r}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.max_seq_len = max_seq_len
        self.max_blocks_per_request = -(-max_seq_len // block_size)

        self.free_blocks: list[int] = list(range(num_blocks))
        self.free_slots: list[int] = list(range(max_cache_slots))
        self.request_to_slot: dict[int, int] = {}
        self._leases: list[_Lease | None] = [None] * max_cache_slots

        self.block_table = t.full((max_cache_slots, self.max_blocks_per_request), -1, dtype=t.int32, device=device)
        self.seq_lens = t.zeros(max_cache_slots, dtype=t.int32, device=device)

    # ----------------------------------------------------------------- queries

    def required_blocks(self, seq_len: int) -> int:
        """Pages that hold `seq_len` tokens; seq_len must lie in [0, max_seq_len]."""
        if not _is_int(seq_len) or seq_len < 0 or seq_len > self.max_seq_len:
            raise ValueError(f"sequence length {seq_len!r} is not an integer in [0, {self.max_seq_len}]")
        return -(-seq_len // self.block_size)

    def check_slot(self, slot: int):
        """ValueError unless `slot` is a slot index owned by some request."""
        self._lease(slot)

    def get_slot(self, request_id: int) -> int:
        return self.request_to_slot[request_id]

    def get_seq_len(self, request_id: int) -> int:
        return self._leases[self.get_slot(request_id)].committed

    def get_block_table(self, slots):
        """Rows of the block table for owned slots."""
        slots = self.indices(slots)
        for slot in slots.reshape(-1).tolist():
            self._lease(slot)
        return self.block_table[slots]

    def _lease(self, slot) -> _Lease:
        if not _is_int(slot) or not 0 <= slot < len(self._leases):
            raise ValueError(f"cache slot {slot!r} is not a slot index")
        lease = self._leases[slot]
        if lease is None:
            raise ValueError(f"cache slot {slot} has no owner")
        return lease

    # ---------------------------------------------------------------- requests

    def allocate_request(self, request_id: int, initial_seq_len: int) -> int:
        """Give `request_id` a slot with room for `initial_seq_len` tokens; returns the slot."""
        if not _is_int(request_id):
            raise ValueError(f"request id {request_id!r} is not an integer")
        if request_id in self.request_to_slot:
            raise ValueError(f"request {request_id} already holds slot {self.request_to_slot[request_id]}")
        pages = self.required_blocks(initial_seq_len)
        if not self.free_slots or pages > len(self.free_blocks):
            raise CacheCapacityError(
                f"no room for request {request_id}: {len(self.free_slots)} free slots, "
                f"{len(self.free_blocks)} free pages, {pages} pages wanted")
        slot = self.free_slots.pop()
        self._leases[slot] = _Lease(request_id)
        self.request_to_slot[request_id] = slot
        self._grow({slot: pages})
        return slot

    def free_request(self, request_id: int):
        """Return the request's pages and slot to the free stacks; reset its table row
        and length on the device (never read back: the host lists are authoritative)."""
        slot = self.get_slot(request_id)
        lease = self._leases[slot]
        self.block_table[slot].fill_(-1)
        self.seq_lens[slot] = 0
        self.free_blocks.extend(lease.pages)
        self._leases[slot] = None
        del self.request_to_slot[request_id]
        self.free_slots.append(slot)

    def clear(self):
        for request_id in list(self.request_to_slot):
            self.free_request(request_id)

    # ---------------------------------------------------------------- capacity

    def reserve_capacity(self, slot: int, required_seq_len: int):
        self.reserve_batch_capacity([slot], [required_seq_len])

    def reserve_batch_capacity(self, slots: Sequence[int], required_seq_lens: Sequence[int]):
        """Grow each slot to hold its required length. All or nothing: if the pool
        cannot cover the whole batch, no page is taken (CacheCapacityError)."""
        if len(slots) != len(required_seq_lens) or len(set(slots)) != len(slots):
            raise ValueError("capacity reservation needs distinct slots, one required length each")
        wanted = {}
        for slot, length in zip(slots, required_seq_lens):
            held = len(self._lease(slot).pages)
            wanted[slot] = max(0, self.required_blocks(length) - held)
        if sum(wanted.values()) > len(self.free_blocks):
            raise CacheCapacityError(
                f"{sum(wanted.values())} pages wanted, {len(self.free_blocks)} free")
        self._grow(wanted)

    def _grow(self, wanted: dict[int, int]):
        """Append pages from the top of the free stack to each slot (the caller has
        checked that there are enough), and publish them in the block table."""
        for slot, count in wanted.items():
            if count == 0:
                continue
            lease = self._leases[slot]
            cut = len(self.free_blocks) - count
            new_pages = self.free_blocks[cut:]
            del self.free_blocks[cut:]
            first = len(lease.pages)
            lease.pages.extend(new_pages)
            self.block_table[slot, first:first + count] = t.tensor(new_pages, dtype=t.int32,
                                                                   device=self.block_table.device)

    # --------------------------------------------------------- committed length

    def advance(self, request_id: int, num_tokens: int):
        self.advance_batch([request_id], [num_tokens])

    def advance_batch(self, request_ids: Sequence[int], num_tokens: Sequence[int]):
        """Commit `num_tokens[i]` more tokens for `request_ids[i]`; refused as a whole if
        any request would pass its reserved pages or max_seq_len."""
        if len(request_ids) != len(num_tokens) or len(set(request_ids)) != len(request_ids):
            raise ValueError("advance needs distinct request ids, one token count each")
        updates = []
        for request_id, count in zip(request_ids, num_tokens):
            if not _is_int(count) or count < 0:
                raise ValueError(f"token count {count!r} is not a nonnegative integer")
            slot = self.get_slot(request_id)
            lease = self._leases[slot]
            length = lease.committed + count
            if length > min(self.max_seq_len, len(lease.pages) * self.block_size):
                raise CacheCapacityError(
                    f"request {request_id} would hold {length} tokens; its pages hold "
                    f"{len(lease.pages) * self.block_size} (max_seq_len {self.max_seq_len})")
            updates.append((slot, length))
        if not updates:
            return
        rows = t.tensor([slot for slot, _ in updates], dtype=t.long, device=self.seq_lens.device)
        self.seq_lens[rows] = t.tensor([n for _, n in updates], dtype=t.int32, device=self.seq_lens.device)
        for slot, length in updates:
            self._leases[slot].committed = length

    # --------------------------------------------------------------- locations

    def indices(self, values) -> t.Tensor:
        """`values` as an int32/int64 tensor on the table's device."""
        out = t.as_tensor(values, device=self.block_table.device)
        if out.dtype not in (t.int32, t.int64):
            raise ValueError(f"cache indices must be int32 or int64, got {out.dtype}")
        return out

    def get_physical_location(self, slots, token_positions, *, validate=True):
        """(page, offset) of each (slot, position): `block_table[slot, pos // BS]`,
        `pos % BS` (slots and positions broadcast). With `validate` the bounds and the
        page's presence are checked, which reads device values (a host sync); runtime
        code that built the metadata itself passes validate=False."""
        slots, positions = t.broadcast_tensors(self.indices(slots), self.indices(token_positions))
        if validate:
            inside = ((slots >= 0) & (slots < self.block_table.shape[0])
                      & (positions >= 0) & (positions < self.max_seq_len))
            if not bool(inside.all()):
                raise ValueError("a cache slot or token position is out of range")
        pages = self.block_table[slots, positions // self.block_size]
        if validate and not bool((pages >= 0).all()):
            raise ValueError("a token position lies outside its slot's reserved pages")
        return pages, positions % self.block_size

    def append_request(self, request_id, token_positions, ks, vs, paged_cache):
        """Write one request's K/V rows at the given positions of its slot."""
        pages, offsets = self.get_physical_location(self.get_slot(request_id), token_positions)
        paged_cache.append_kv(pages, offsets, ks, vs)

    def resolve_batch_locations(self, cache_slots, cu_seqlens, token_positions, *, validate=True):
        """Write locations of a packed batch: token i of sequence b (tokens
        cu_seqlens[b] .. cu_seqlens[b + 1] - 1) goes to position token_positions[i] of
        slot cache_slots[b]."""
        device = self.block_table.device
        if any(x.device != device for x in (cache_slots, cu_seqlens, token_positions)):
            raise ValueError(f"batch metadata must be on the cache device {device}")
        batch = cache_slots.numel()
        if cache_slots.ndim != 1 or token_positions.ndim != 1 or cu_seqlens.shape != (batch + 1,):
            raise ValueError("packed batch metadata needs cache_slots [B], cu_seqlens [B + 1], positions [T]")
        counts = cu_seqlens[1:] - cu_seqlens[:-1]
        if validate:
            total = token_positions.numel()
            if int(cu_seqlens[0]) != 0 or int(cu_seqlens[-1]) != total or not bool((counts > 0).all()):
                raise ValueError("cu_seqlens must start at 0, end at the token count and increase strictly")
        per_token_slot = t.repeat_interleave(cache_slots, counts, output_size=token_positions.numel())
        return self.get_physical_location(per_token_slot, token_positions, validate=validate)

    def create_container(self, cache_slots, cu_seqlens, token_positions, *, validate=True):
        """The batch's CacheContainer, built before its tokens are committed: each
        sequence attends over its committed tokens plus this batch's
        (`context_lengths = seq_lens[slot] + tokens`, reference `:347`).

        With `validate` (which reads device values) the container is also marked
        `appends_last_position` when every sequence brings one token at its committed
        length. validate=False is for metadata the runtime built itself; it never
        synchronizes and leaves the mark off."""
        blocks, offsets = self.resolve_batch_locations(cache_slots, cu_seqlens, token_positions, validate=validate)
        committed = self.seq_lens[cache_slots]
        counts = cu_seqlens[1:] - cu_seqlens[:-1]
        last = False
        if validate and token_positions.numel() == cache_slots.numel():
            last = bool((token_positions == committed).all())
        return CacheContainer(cache_slots, blocks, offsets, committed + counts, self.block_table, last)
