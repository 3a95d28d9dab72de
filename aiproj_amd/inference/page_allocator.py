"""Page and slot ownership with a device mirror of the kernel metadata.

Reference `src/torch_llm/inference/page_allocator.py:9-366`: same classes, methods,
argument meaning, allocation order and error types.

* The CPU lists are authoritative (`free_blocks`, `slot_blocks`, `slot_seq_lens` ...).
* The device mirrors are what the kernels read:
  `block_table [max_cache_slots, ceil(max_seq_len / block_size)]` int32, -1 when
  unallocated, and `seq_lens [max_cache_slots]` int32 (committed lengths).
* Capacity is reserved separately from committed length; a batch reservation is
  all-or-nothing (`CacheCapacityError`).
* One owning thread and stream; no locking.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch as t

from aiproj_amd.inference.paged_kv_cache import PagedKVCache


class CacheCapacityError(RuntimeError):
    """The cache pool cannot satisfy an otherwise valid allocation."""


def _positive_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool) and value > 0


def _plain_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def initialize_cache(kvcache_config, model_config, device):
    """One shared allocator and independent K/V storage per layer (reference `:13-36`)."""
    manager = PageAllocator(
        kvcache_config.num_blocks,
        kvcache_config.block_size,
        kvcache_config.max_cache_slots,
        kvcache_config.cache_max_seq_len,
        device,
    )
    caches = [
        PagedKVCache(
            kvcache_config.num_blocks,
            kvcache_config.block_size,
            model_config.num_kv_heads,
            model_config.head_dim,
            device,
            cache_dtype=kvcache_config.kv_cache_dtype,
            scale_dtype=kvcache_config.kv_scale_dtype,
        )
        for _ in range(model_config.num_layers)
    ]
    return manager, caches


@dataclass
class CacheContainer:
    """Per-batch cache metadata handed to the model (reference `:358-366`)."""

    cache_slots: t.Tensor
    physical_blocks: t.Tensor
    block_offsets: t.Tensor
    context_lengths: t.Tensor
    # Full table, indexed by the persistent cache_slots inside the decode kernel.
    block_table: t.Tensor


class PageAllocator:
    """Own page allocation on the CPU and mirror kernel metadata on the device."""

    def __init__(self, num_blocks, block_size, max_cache_slots, max_seq_len, device):
        for name, value in (
            ("num_blocks", num_blocks),
            ("block_size", block_size),
            ("max_cache_slots", max_cache_slots),
            ("max_seq_len", max_seq_len),
        ):
            if not _positive_int(value):
                raise ValueError(f"{name} must be a positive integer")

        self.num_blocks = num_blocks
        self.block_size = block_size
        self.max_seq_len = max_seq_len
        self.max_blocks_per_request = -(-max_seq_len // block_size)

        # Pages are handed out from the end of the free list and returned to its end.
        self.free_blocks = list(range(num_blocks))
        self.free_slots = list(range(max_cache_slots))
        self.request_to_slot: dict[int, int] = {}

        self.block_table = t.full((max_cache_slots, self.max_blocks_per_request), -1,
                                  dtype=t.int32, device=device)
        self.seq_lens = t.zeros(max_cache_slots, dtype=t.int32, device=device)

        self.slot_num_blocks = [0] * max_cache_slots
        self.slot_requests: list[int | None] = [None] * max_cache_slots
        self.slot_blocks: list[list[int]] = [[] for _ in range(max_cache_slots)]
        self.slot_seq_lens = [0] * max_cache_slots

    # -- capacity ----------------------------------------------------------

    def required_blocks(self, seq_len: int) -> int:
        if not _plain_int(seq_len) or not 0 <= seq_len <= self.max_seq_len:
            raise ValueError(f"Sequence length must be an integer in [0, {self.max_seq_len}]")
        return -(-seq_len // self.block_size)

    def check_slot(self, slot: int):
        if not _plain_int(slot) or not 0 <= slot < len(self.slot_requests):
            raise ValueError("Invalid cache slot")
        if self.slot_requests[slot] is None:
            raise ValueError(f"Cache slot {slot} is not allocated")

    def allocate_request(self, request_id: int, initial_seq_len: int) -> int:
        if not _plain_int(request_id):
            raise ValueError("request_id must be an integer")
        if request_id in self.request_to_slot:
            raise ValueError(f"Request {request_id} already owns a cache slot")
        needed = self.required_blocks(initial_seq_len)
        if not self.free_slots or needed > len(self.free_blocks):
            raise CacheCapacityError("Insufficient cache slots or blocks")

        slot = self.free_slots.pop()
        self.request_to_slot[request_id] = slot
        self.slot_requests[slot] = request_id
        try:
            self.reserve_capacity(slot, initial_seq_len)
        except Exception:
            self.free_request(request_id)
            raise
        return slot

    def reserve_capacity(self, slot: int, required_seq_len: int):
        self.reserve_batch_capacity([slot], [required_seq_len])

    def reserve_batch_capacity(self, slots: Sequence[int], required_seq_lens: Sequence[int]):
        """Check the whole batch before taking any page from the free pool."""
        if len(slots) != len(required_seq_lens) or len(set(slots)) != len(slots):
            raise ValueError("Capacity reservations require one length per unique slot")

        plan = []
        for slot, length in zip(slots, required_seq_lens):
            self.check_slot(slot)
            plan.append((slot, max(0, self.required_blocks(length) - self.slot_num_blocks[slot])))
        if sum(count for _, count in plan) > len(self.free_blocks):
            raise CacheCapacityError("Insufficient cache blocks")

        for slot, count in plan:
            if count == 0:
                continue
            taken = self.free_blocks[-count:]
            del self.free_blocks[-count:]
            first = self.slot_num_blocks[slot]
            self.block_table[slot, first:first + count] = t.tensor(
                taken, dtype=t.int32, device=self.block_table.device)
            self.slot_blocks[slot].extend(taken)
            self.slot_num_blocks[slot] += count

    # -- committed lengths ---------------------------------------------------

    def advance(self, request_id: int, num_tokens: int):
        self.advance_batch([request_id], [num_tokens])

    def advance_batch(self, request_ids: Sequence[int], num_tokens: Sequence[int]):
        if len(request_ids) != len(num_tokens) or len(set(request_ids)) != len(request_ids):
            raise ValueError("Advancing requires one token count per unique request")

        slots, lengths = [], []
        for request_id, count in zip(request_ids, num_tokens):
            if not _plain_int(count) or count < 0:
                raise ValueError("num_tokens must be a nonnegative integer")
            slot = self.get_slot(request_id)
            length = self.slot_seq_lens[slot] + count
            if length > self.max_seq_len or length > self.slot_num_blocks[slot] * self.block_size:
                raise CacheCapacityError("Sequence exceeds its reserved cache capacity")
            slots.append(slot)
            lengths.append(length)

        if slots:
            device = self.seq_lens.device
            self.seq_lens[t.tensor(slots, device=device, dtype=t.long)] = t.tensor(
                lengths, device=device, dtype=t.int32)
            for slot, length in zip(slots, lengths):
                self.slot_seq_lens[slot] = length

    def get_slot(self, request_id: int) -> int:
        return self.request_to_slot[request_id]

    def get_seq_len(self, request_id: int) -> int:
        return self.slot_seq_lens[self.get_slot(request_id)]

    # -- locations -------------------------------------------------------------

    def indices(self, values) -> t.Tensor:
        values = t.as_tensor(values, device=self.block_table.device)
        if values.dtype not in (t.int32, t.int64):
            raise ValueError("Cache indices must be int32 or int64")
        return values

    def get_physical_location(self, slots, token_positions, *, validate=True):
        """Page-table gather for writes: (block_table[slot, pos // BS], pos % BS).

        With validate=True the bounds checks read device values (a host sync);
        the runtime passes validate=False for metadata it built itself.
        """
        slots = self.indices(slots)
        token_positions = self.indices(token_positions)
        slots, token_positions = t.broadcast_tensors(slots, token_positions)

        if validate:
            in_range = (
                (slots >= 0)
                & (slots < self.block_table.shape[0])
                & (token_positions >= 0)
                & (token_positions < self.max_seq_len)
            )
            if not bool(in_range.all()):
                raise ValueError("Cache slots or token positions are out of bounds")

        physical_blocks = self.block_table[slots, token_positions // self.block_size]
        if validate and not bool((physical_blocks >= 0).all()):
            raise ValueError("Token position has no reserved cache block")
        return physical_blocks, token_positions % self.block_size

    # -- release -----------------------------------------------------------------

    def free_request(self, request_id: int):
        slot = self.get_slot(request_id)
        # CPU ownership is authoritative: the device row is reset, never read back.
        self.block_table[slot].fill_(-1)
        self.seq_lens[slot] = 0

        self.free_blocks.extend(self.slot_blocks[slot])
        self.slot_blocks[slot] = []
        self.slot_num_blocks[slot] = 0
        self.slot_seq_lens[slot] = 0
        self.slot_requests[slot] = None
        del self.request_to_slot[request_id]
        self.free_slots.append(slot)

    def clear(self):
        for request_id in list(self.request_to_slot):
            self.free_request(request_id)

    def get_block_table(self, slots):
        slots = self.indices(slots)
        for slot in slots.reshape(-1).tolist():
            self.check_slot(slot)
        return self.block_table[slots]

    # -- batch helpers ---------------------------------------------------------------

    def append_request(self, request_id, token_positions, ks, vs, paged_cache):
        blocks, offsets = self.get_physical_location(self.get_slot(request_id), token_positions)
        paged_cache.append_kv(blocks, offsets, ks, vs)

    def resolve_batch_locations(self, cache_slots, cu_seqlens, token_positions, *, validate=True):
        if not (cache_slots.device == cu_seqlens.device == token_positions.device
                == self.block_table.device):
            raise ValueError("Batch metadata and cache must be on the same device")
        if (
            cache_slots.ndim != 1
            or cu_seqlens.shape != (cache_slots.numel() + 1,)
            or token_positions.ndim != 1
        ):
            raise ValueError("Invalid packed batch metadata shapes")

        per_sequence = cu_seqlens[1:] - cu_seqlens[:-1]
        if validate and (
            int(cu_seqlens[0]) != 0
            or int(cu_seqlens[-1]) != token_positions.numel()
            or not bool((per_sequence > 0).all())
        ):
            raise ValueError("Invalid cumulative sequence lengths")

        token_slots = t.repeat_interleave(cache_slots, per_sequence, output_size=token_positions.numel())
        return self.get_physical_location(token_slots, token_positions, validate=validate)

    def create_container(self, cache_slots, cu_seqlens, token_positions, *, validate=True):
        """Write locations plus the full attention context, before the batch is committed.

        context_lengths = committed length + tokens of this batch (reference `:347`).
        """
        physical_blocks, block_offsets = self.resolve_batch_locations(
            cache_slots, cu_seqlens, token_positions, validate=validate)
        context_lengths = self.seq_lens[cache_slots] + cu_seqlens[1:] - cu_seqlens[:-1]
        return CacheContainer(cache_slots, physical_blocks, block_offsets, context_lengths, self.block_table)
