"""KV runtime state and the KernelIR executor of the gfx950 backend.

``PreallocatedKVCacheState`` keeps the reference's contract
(src/stateful_llm_compiler/execution.py:98-475): per-layer physical buffers
B x capacity x H x D (contiguous_bshd) that never move, int64 lengths per
batch row, immutable SSA versions (``advance`` returns a new state sharing
the buffers), validation errors as ``ExecutionError``.  Its writer / runner
plug-ins are the HIP kernels; the capacity guard is a device-side flag (no
host synchronisation on the hot path) read by ``check_capacity()``.

``HipExecutor`` walks a lowered KernelIR function and dispatches each op by
name (triton_executor.py:69-130 in the reference), validating every argument
and result against its IR type like the reference executor
(execution.py:530-579, 1094-1157).  It executes only lowered ops: an
unlowered ``serve.*`` / ``aten.*`` op raises instead of falling back to eager
PyTorch.
"""

from __future__ import annotations

import re
import weakref
from dataclasses import dataclass, replace
from typing import Any, Callable, Sequence

import torch
import torch.nn.functional as F

from .backends import (
    hip_add,
    hip_decode_attention,
    hip_rope_decode_attention,
    hip_embedding,
    hip_kv_advance,
    hip_kv_store,
    hip_linear,
    hip_linear_residual,
    hip_norm_linear_group,
    hip_norm_linear_swiglu,
    hip_paged_decode_attention,
    hip_paged_kv_store,
    hip_paged_rope_decode_attention,
    hip_prefill_attention,
    hip_prefill_mask_tiles,
    hip_rms_norm,
    hip_rope,
    hip_rope_kv_store,
    hip_rope_table,
    hip_swiglu,
)
from . import _native
from .backends.hip_attention import exact_max_tokens
from .cost_model import choose_variant, linear_tile, split_tokens, waves_per_row
from .ir import (
    Function,
    IRType,
    KVStateType,
    Module,
    ScalarType,
    StaticDim,
    SymbolicDim,
    TensorType,
    TupleType,
    UnknownType,
)
from .lowering import require_full_lowering


class ExecutionError(RuntimeError):
    pass


DTYPES = {
    "f16": torch.float16,
    "bf16": torch.bfloat16,
    "f32": torch.float32,
    "f64": torch.float64,
    "i8": torch.int8,
    "i16": torch.int16,
    "i32": torch.int32,
    "i64": torch.int64,
    "i1": torch.bool,
}
DTYPE_NAMES = {value: key for key, value in DTYPES.items()}


def _zeroed_layers(count: int, shape: tuple[int, ...], device, dtype, *, pairs: bool = False):
    """``count`` zeroed per-layer tensors of ``shape`` as views of one
    allocation, so that a whole state is cleared by one fill instead of one
    launch per layer and tensor.  ``pairs``: the first half of the views
    (keys) and the second half (values) as two tuples."""

    block = torch.zeros((count, *shape), device=device, dtype=dtype)
    views = tuple(block[i] for i in range(count))
    if pairs:
        half = count // 2
        return views[:half], views[half:]
    return (views,)


@dataclass(frozen=True)
class PreallocatedKVCacheState:
    """Shared physical KV buffers plus per-version logical lengths."""

    keys: tuple[torch.Tensor, ...]
    values: tuple[torch.Tensor, ...]
    lengths: tuple[torch.Tensor, ...]
    capacity: int
    generation: int = 0
    # int32[1] device flag shared by all versions: set when a store or an
    # advance leaves [0, capacity].
    overflow: torch.Tensor | None = None
    # When true, advance() updates the lengths tensors in place (stable
    # addresses for HIP graph replay); otherwise it creates new tensors.
    in_place_lengths: bool = False
    # Slots whose lengths are known (on the host) to be zero, so prefill_store
    # needs no device-to-host check; None = unknown.
    zero_slots: frozenset[int] | None = None
    # Device scratch (arrival counters, split partials) of the kernels this
    # state runs, shared by all versions: one state's kernels run in order on
    # one stream, and two states (two decoders) never share it.  None = the
    # current stream's workspace.
    workspace: _native.DeviceWorkspace | None = None

    def __post_init__(self) -> None:
        if self.capacity <= 0:
            raise ExecutionError("KV capacity must be positive")
        if not self.keys or len(self.keys) != len(self.values) or len(self.keys) != len(self.lengths):
            raise ExecutionError("KV key/value/length slot counts must agree")
        for key, value, lengths in zip(self.keys, self.values, self.lengths):
            if key.shape != value.shape or key.ndim != 4:
                raise ExecutionError("KV buffers must be equal-shaped B x C x H x D tensors")
            if key.shape[1] != self.capacity:
                raise ExecutionError("KV buffer dim 1 must equal the capacity")
            if lengths.shape != (key.shape[0],):
                raise ExecutionError("KV lengths must be a 1-D batch tensor")
            if lengths.dtype != torch.int64:
                raise ExecutionError("KV lengths must be int64")

    @classmethod
    def empty_from_key_template(
        cls, key: torch.Tensor, *, num_layers: int, capacity: int, in_place_lengths: bool = False
    ) -> "PreallocatedKVCacheState":
        """Zeroed buffers for every layer from a B x H x T x D key template."""

        if key.ndim != 4 or num_layers <= 0 or capacity <= 0:
            raise ExecutionError("KV init got an illegal template, layer count or capacity")
        batch, heads, _, head_dim = key.shape
        keys, values = _zeroed_layers(2 * num_layers, (batch, capacity, heads, head_dim),
                                      key.device, key.dtype, pairs=True)
        (lengths,) = _zeroed_layers(num_layers, (batch,), key.device, torch.int64)
        overflow = torch.zeros(1, device=key.device, dtype=torch.int32)
        return cls(keys, values, lengths, capacity, overflow=overflow,
                   in_place_lengths=in_place_lengths, zero_slots=frozenset(range(num_layers)),
                   workspace=_device_workspace(key.device))

    @classmethod
    def from_layer_tensors(
        cls,
        past_key_values: Sequence[tuple[torch.Tensor, torch.Tensor]],
        *,
        capacity: int,
        in_place_lengths: bool = False,
    ) -> "PreallocatedKVCacheState":
        """Copy logical B x H x S x D caches into preallocated slots (setup only)."""

        if not past_key_values:
            raise ExecutionError("a multi-layer KV cache needs at least one slot")
        keys, values, lengths = [], [], []
        structure = None
        for slot, (key, value) in enumerate(past_key_values):
            if key.shape != value.shape or key.ndim != 4:
                raise ExecutionError(f"layer {slot}: initial K/V must be equal B x H x S x D tensors")
            batch, heads, sequence, head_dim = key.shape
            this = (batch, heads, sequence, head_dim, key.dtype, key.device)
            if structure is None:
                structure = this
            elif this != structure:
                raise ExecutionError("all layer slots need one K/V shape, dtype and device")
            if sequence > capacity:
                raise ExecutionError(f"layer {slot}: initial length {sequence} exceeds capacity {capacity}")
            kb = torch.zeros(batch, capacity, heads, head_dim, device=key.device, dtype=key.dtype)
            vb = torch.zeros_like(kb)
            kb[:, :sequence].copy_(key.transpose(1, 2))
            vb[:, :sequence].copy_(value.transpose(1, 2))
            keys.append(kb)
            values.append(vb)
            lengths.append(torch.full((batch,), sequence, device=key.device, dtype=torch.int64))
        overflow = torch.zeros(1, device=keys[0].device, dtype=torch.int32)
        return cls(tuple(keys), tuple(values), tuple(lengths), capacity, overflow=overflow,
                   in_place_lengths=in_place_lengths, workspace=_device_workspace(keys[0].device))

    def positions(self, slot: int) -> torch.Tensor:
        try:
            return self.lengths[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error

    def read(self, slot: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Logical B x H x S x D view of the longest prefix (host sync)."""

        try:
            key, value, lengths = self.keys[slot], self.values[slot], self.lengths[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error
        used = int(lengths.max().item())
        return key[:, :used].transpose(1, 2), value[:, :used].transpose(1, 2)

    def decode_attention(
        self,
        slot: int,
        query: torch.Tensor,
        attention_mask: torch.Tensor,
        *,
        groups: int,
        scale: float,
        runner: Callable[..., torch.Tensor] = hip_decode_attention,
        softmax_order: str = "online",
        split_tokens: int = 0,
    ) -> torch.Tensor:
        """Decode attention straight from the B x Capacity x H x D buffers.

        A custom ``runner`` is called as the reference calls it
        (``runner(query, key_buffer, value_buffer, lengths, mask, scale=)``);
        the HIP runner also gets this state's workspace, the softmax order
        (the exact order where the mask fits it, else the online one) and the
        split a profile plan chose."""

        key_buffer, value_buffer, lengths = self._attention_inputs(slot, query, attention_mask, groups)
        if runner is not hip_decode_attention:
            return runner(query, key_buffer, value_buffer, lengths, attention_mask, scale=scale)
        order = attention_order(softmax_order, attention_mask.shape[-1], query)
        return runner(query, key_buffer, value_buffer, lengths,
                      _kernel_mask(attention_mask, self.capacity), scale=scale,
                      softmax_order=order, workspace=self.workspace, split_tokens=split_tokens)

    def _attention_inputs(self, slot, query, attention_mask, groups):
        try:
            key_buffer, value_buffer, lengths = self.keys[slot], self.values[slot], self.lengths[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error
        if query.ndim != 4 or query.shape[2] != 1:
            raise ExecutionError("decode attention query must be B x H x 1 x D")
        if attention_mask.ndim != 4 or attention_mask.shape[2] != 1:
            raise ExecutionError("decode attention mask must be B x 1 x 1 x S")
        if (
            query.shape[0] != key_buffer.shape[0]
            or query.shape[0] != attention_mask.shape[0]
            or query.shape[3] != key_buffer.shape[3]
        ):
            raise ExecutionError("decode attention batch or head dim does not match the KV buffer")
        if groups <= 0 or query.shape[1] != key_buffer.shape[2] * groups:
            raise ExecutionError("decode attention GQA groups do not match")
        if attention_mask.shape[-1] > self.capacity:
            raise ExecutionError("decode attention mask is longer than the KV capacity")
        return key_buffer, value_buffer, lengths

    def store(
        self,
        slot: int,
        key: torch.Tensor,
        value: torch.Tensor,
        positions: torch.Tensor,
        *,
        writer: Callable[..., None] = hip_kv_store,
    ) -> "PreallocatedKVCacheState":
        buffer_key, buffer_value = self._validate_store(slot, key, value, positions)
        writer(buffer_key, buffer_value, key, value, positions, overflow=self.overflow)
        # Only rows past the current logical length change: older versions'
        # visible prefixes are untouched, so the same object is returned.
        return self

    def rope_store(
        self,
        slot: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        cosine: torch.Tensor,
        sine: torch.Tensor,
        positions: torch.Tensor,
    ) -> tuple[torch.Tensor, "PreallocatedKVCacheState"]:
        """RoPE of ``query``/``key`` with the rotated key and ``value`` stored
        at ``positions`` in one kernel: the rotated query and this state."""

        buffer_key, buffer_value = self._validate_store(slot, key, value, positions)
        q_rot = hip_rope_kv_store(query, key, value, cosine, sine, buffer_key, buffer_value,
                                  positions, overflow=self.overflow)
        return q_rot, self

    def rope_store_advance(
        self,
        slot: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        cosine: torch.Tensor,
        sine: torch.Tensor,
        *,
        delta: int,
    ) -> tuple[torch.Tensor, "PreallocatedKVCacheState"]:
        """``rope_store`` at this slot's lengths followed by ``advance(slot,
        delta)``, in one kernel: the rotated query and the advanced state."""

        if delta <= 0:
            raise ExecutionError("KV advance delta must be positive")
        positions = self.positions(slot)
        buffer_key, buffer_value = self._validate_store(slot, key, value, positions)
        out = positions if self.in_place_lengths else torch.empty_like(positions)
        q_rot = hip_rope_kv_store(query, key, value, cosine, sine, buffer_key, buffer_value,
                                  positions, overflow=self.overflow, advance=delta, lengths_out=out,
                                  workspace=self.workspace)
        lengths = list(self.lengths)
        lengths[slot] = out
        zero = None if self.zero_slots is None else self.zero_slots - {slot}
        return q_rot, replace(self, lengths=tuple(lengths), generation=self.generation + 1,
                              zero_slots=zero)

    def rope_store_attention(
        self,
        slot: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        cosine: torch.Tensor,
        sine: torch.Tensor,
        attention_mask: torch.Tensor,
        *,
        groups: int,
        scale: float,
        softmax_order: str = "online",
    ) -> tuple[torch.Tensor, "PreallocatedKVCacheState"]:
        """``rope_store_advance(slot, ..., delta=1)`` then ``decode_attention``
        of the rotated query over the advanced state, in one kernel where it
        takes the case (else the two ops): the attention output and the
        advanced state."""

        positions = self.positions(slot)
        buffer_key, buffer_value = self._validate_store(slot, key, value, positions)
        self._attention_inputs(slot, query, attention_mask, groups)
        out = positions if self.in_place_lengths else torch.empty_like(positions)
        result = None
        if key.shape[2] == 1:
            result = hip_rope_decode_attention(
                query, key, value, cosine, sine, buffer_key, buffer_value, positions, out,
                _kernel_mask(attention_mask, self.capacity), scale=scale, overflow=self.overflow,
                softmax_order=attention_order(softmax_order, attention_mask.shape[-1], query),
                workspace=self.workspace,
            )
        if result is None:
            q_rot, state = self.rope_store_advance(slot, query, key, value, cosine, sine, delta=1)
            return state.decode_attention(slot, q_rot, attention_mask, groups=groups,
                                          scale=scale, softmax_order=softmax_order), state
        lengths = list(self.lengths)
        lengths[slot] = out
        zero = None if self.zero_slots is None else self.zero_slots - {slot}
        return result, replace(self, lengths=tuple(lengths), generation=self.generation + 1,
                               zero_slots=zero)

    def prefill_store(
        self,
        slot: int,
        key: torch.Tensor,
        value: torch.Tensor,
        *,
        writer: Callable[..., None] = hip_kv_store,
    ) -> "PreallocatedKVCacheState":
        """Write a layer's prompt K/V from position 0, then advance by T."""

        positions = self.positions(slot)
        if self.zero_slots is not None:
            if slot not in self.zero_slots:
                raise ExecutionError("prefill KV store needs the slot's length to be 0")
        elif bool((positions != 0).any()):
            raise ExecutionError("prefill KV store needs the slot's length to be 0")
        self.store(slot, key, value, positions, writer=writer)
        return self.advance(slot, delta=key.shape[2])

    def advance(self, slot: int, *, delta: int) -> "PreallocatedKVCacheState":
        if delta <= 0:
            raise ExecutionError("KV advance delta must be positive")
        positions = self.positions(slot)
        out = positions if self.in_place_lengths else None
        next_lengths = hip_kv_advance(positions, delta, self.capacity, out=out, overflow=self.overflow)
        lengths = list(self.lengths)
        lengths[slot] = next_lengths
        zero = None if self.zero_slots is None else self.zero_slots - {slot}
        return replace(self, lengths=tuple(lengths), generation=self.generation + 1, zero_slots=zero)

    def check_capacity(self) -> None:
        """Synchronise and raise if any store or advance overflowed the capacity."""

        if self.overflow is not None and int(self.overflow.item()) != 0:
            raise ExecutionError(f"KV store or advance exceeded capacity {self.capacity}")

    def _validate_store(self, slot, key, value, positions):
        try:
            buffer_key, buffer_value = self.keys[slot], self.values[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error
        if key.shape != value.shape or key.ndim != 4:
            raise ExecutionError("KV store K/V must be equal B x H x T x D tensors")
        batch, heads, _, head_dim = key.shape
        if batch != buffer_key.shape[0] or heads != buffer_key.shape[2] or head_dim != buffer_key.shape[3]:
            raise ExecutionError("KV store batch, heads or head dim does not match")
        if positions.shape != (batch,) or positions.dtype != torch.int64:
            raise ExecutionError("KV store positions must be a 1-D batch int64 tensor")
        if positions.device != key.device:
            raise ExecutionError("KV store positions and K/V must share a device")
        return buffer_key, buffer_value


def _page_order(batch: int, pages_per_seq: int, device) -> torch.Tensor:
    """Block table of a fully provisioned pool: page j of sequence b is pool
    page j * batch + b, so every sequence's pages are scattered over the pool
    (what a page allocator produces after sequences have grown in turn)."""

    pages = torch.arange(pages_per_seq, dtype=torch.int32).view(1, -1) * batch
    return (pages + torch.arange(batch, dtype=torch.int32).view(-1, 1)).to(device)


@dataclass(frozen=True)
class PagedKVCacheState(PreallocatedKVCacheState):
    """The paged KV layout (``KVStateType.layout == "paged"``): the next step
    the reference plans after its contiguous buffers
    (docs/kv-bufferization.md:317-323).

    ``keys``/``values`` hold one page pool per layer, [num_pages,
    page_tokens, H, D]; ``block_table`` (int32 [B, capacity / page_tokens],
    shared by every layer) names the pool page of each sequence's tokens
    [j * page_tokens, (j + 1) * page_tokens).  Lengths, versions, the overflow
    flag and the workspace behave as in the contiguous state, and every op
    gives the contiguous state's result bit for bit.  The model's decode step
    (RoPE, store, advance, attention) runs as one paged kernel like the
    contiguous one; RoPE + store alone runs as two kernels.

    One stream per state: every version of a state shares one device
    workspace (arrival counters, split partials), so the state's kernels
    must run in order on one stream (or inside one captured graph).  The
    block table is checked once at construction (device and entry range).
    """

    block_table: torch.Tensor | None = None
    page_tokens: int = 0

    def __post_init__(self) -> None:
        if self.capacity <= 0:
            raise ExecutionError("KV capacity must be positive")
        p = self.page_tokens
        if p < 16 or p & (p - 1) or self.capacity % p:
            raise ExecutionError("page_tokens must be a power of two >= 16 dividing the capacity")
        table = self.block_table
        if table is None or table.ndim != 2 or table.dtype != torch.int32:
            raise ExecutionError("a paged KV state needs an int32 [B, pages] block table")
        if table.shape[1] != self.capacity // p:
            raise ExecutionError("block table width must be capacity / page_tokens")
        if not self.keys or len(self.keys) != len(self.values) or len(self.keys) != len(self.lengths):
            raise ExecutionError("KV key/value/length slot counts must agree")
        for key, value, lengths in zip(self.keys, self.values, self.lengths):
            if key.shape != value.shape or key.ndim != 4 or key.shape[1] != p:
                raise ExecutionError("KV pools must be equal-shaped pages x page_tokens x H x D tensors")
            if lengths.shape != (table.shape[0],) or lengths.dtype != torch.int64:
                raise ExecutionError("KV lengths must be an int64 [B] tensor")
        self._check_block_table(table, self.keys[0])

    # Tables already checked against a pool size (every state version of one
    # sequence set shares its table, so the host read happens once).
    # id(table) -> (weak reference, pool pages); not a field (no annotation).
    _checked_tables = {}

    @classmethod
    def _check_block_table(cls, table: torch.Tensor, pool: torch.Tensor) -> None:
        """The kernels take every entry as a raw pool page index: check once,
        on the host, that the table lives with the pools and that every entry
        is in [0, pool pages)."""

        if table.device != pool.device:
            raise ExecutionError("the block table must be on the KV pools' device")
        pages = pool.shape[0]
        seen = cls._checked_tables.get(id(table))
        if seen is not None and seen[0]() is table and seen[1] == pages:
            return
        if table.numel() and (int(table.min()) < 0 or int(table.max()) >= pages):
            raise ExecutionError(f"block table entries must be pool page indices in [0, {pages})")
        key = id(table)
        cls._checked_tables[key] = (weakref.ref(table, lambda _, key=key: cls._checked_tables.pop(key, None)),
                                    pages)

    @classmethod
    def empty_from_key_template(
        cls, key: torch.Tensor, *, num_layers: int, capacity: int, in_place_lengths: bool = False,
        page_tokens: int = 64,
    ) -> "PagedKVCacheState":
        """Zeroed pools for every layer from a B x H x T x D key template,
        with capacity / page_tokens pages per sequence."""

        if key.ndim != 4 or num_layers <= 0 or capacity <= 0 or page_tokens <= 0 or capacity % page_tokens:
            raise ExecutionError("paged KV init got an illegal template, layer count, capacity or page size")
        batch, heads, _, head_dim = key.shape
        pages = capacity // page_tokens
        keys, values = _zeroed_layers(2 * num_layers, (batch * pages, page_tokens, heads, head_dim),
                                      key.device, key.dtype, pairs=True)
        (lengths,) = _zeroed_layers(num_layers, (batch,), key.device, torch.int64)
        return cls(keys, values, lengths, capacity,
                   overflow=torch.zeros(1, device=key.device, dtype=torch.int32),
                   in_place_lengths=in_place_lengths, zero_slots=frozenset(range(num_layers)),
                   workspace=_device_workspace(key.device),
                   block_table=_page_order(batch, pages, key.device), page_tokens=page_tokens)

    @classmethod
    def from_layer_tensors(cls, past_key_values, *, capacity: int, in_place_lengths: bool = False,
                           page_tokens: int = 64) -> "PagedKVCacheState":
        """Copy logical B x H x S x D caches into freshly paged slots (setup only)."""

        if not past_key_values:
            raise ExecutionError("a multi-layer KV cache needs at least one slot")
        state = cls.empty_from_key_template(past_key_values[0][0], num_layers=len(past_key_values),
                                            capacity=capacity, in_place_lengths=in_place_lengths,
                                            page_tokens=page_tokens)
        lengths = []
        for slot, (key, value) in enumerate(past_key_values):
            if key.shape != value.shape or key.shape != past_key_values[0][0].shape:
                raise ExecutionError("all layer slots need one K/V shape")
            if key.shape[2] > capacity:
                raise ExecutionError(f"layer {slot}: initial length {key.shape[2]} exceeds capacity {capacity}")
            zero = torch.zeros(key.shape[0], dtype=torch.int64, device=key.device)
            hip_paged_kv_store(state.keys[slot], state.values[slot], state.block_table,
                               key.to(state.keys[slot].dtype), value.to(state.keys[slot].dtype), zero)
            lengths.append(torch.full_like(zero, key.shape[2]))
        return replace(state, lengths=tuple(lengths), zero_slots=None)

    @property
    def batch(self) -> int:
        return self.block_table.shape[0]

    def gather(self, slot: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The contiguous B x capacity x H x D buffers the pages stand for
        (a copy; for eager composites and inspection)."""

        try:
            pools = self.keys[slot], self.values[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error
        index = self.block_table.long()
        return tuple(pool[index].reshape(self.batch, self.capacity, *pool.shape[2:]) for pool in pools)

    def read(self, slot: int) -> tuple[torch.Tensor, torch.Tensor]:
        key, value = self.gather(slot)
        used = int(self.positions(slot).max().item())
        return key[:, :used].transpose(1, 2), value[:, :used].transpose(1, 2)

    def _check_attention(self, slot, query, attention_mask, groups):
        try:
            pool, lengths = self.keys[slot], self.lengths[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error
        if query.ndim != 4 or query.shape[2] != 1:
            raise ExecutionError("decode attention query must be B x H x 1 x D")
        if attention_mask.ndim != 4 or attention_mask.shape[2] != 1:
            raise ExecutionError("decode attention mask must be B x 1 x 1 x S")
        if (query.shape[0] != self.batch or query.shape[0] != attention_mask.shape[0]
                or query.shape[3] != pool.shape[3]):
            raise ExecutionError("decode attention batch or head dim does not match the KV pages")
        if groups <= 0 or query.shape[1] != pool.shape[2] * groups:
            raise ExecutionError("decode attention GQA groups do not match")
        if attention_mask.shape[-1] > self.capacity:
            raise ExecutionError("decode attention mask is longer than the KV capacity")
        return lengths

    def _attention_inputs(self, slot, query, attention_mask, groups):
        # Eager composites read the gathered contiguous buffers.
        lengths = self._check_attention(slot, query, attention_mask, groups)
        key, value = self.gather(slot)
        return key, value, lengths

    def decode_attention(self, slot, query, attention_mask, *, groups, scale,
                         runner=hip_decode_attention, softmax_order="online", split_tokens=0):
        """Decode attention straight from the pages through the block table;
        a custom ``runner`` gets the gathered contiguous buffers."""

        if runner is not hip_decode_attention:
            key, value, lengths = self._attention_inputs(slot, query, attention_mask, groups)
            return runner(query, key, value, lengths, attention_mask, scale=scale)
        lengths = self._check_attention(slot, query, attention_mask, groups)
        order = attention_order(softmax_order, attention_mask.shape[-1], query)
        return hip_paged_decode_attention(
            query, self.keys[slot], self.values[slot], self.block_table, lengths,
            _kernel_mask(attention_mask, self.capacity),
            scale=scale, softmax_order=order, workspace=self.workspace, split_tokens=split_tokens)

    def _validate_store(self, slot, key, value, positions):
        try:
            pool_key, pool_value = self.keys[slot], self.values[slot]
        except IndexError as error:
            raise ExecutionError(f"KV buffer has no slot {slot}") from error
        if key.shape != value.shape or key.ndim != 4:
            raise ExecutionError("KV store K/V must be equal B x H x T x D tensors")
        batch, heads, _, head_dim = key.shape
        if batch != self.batch or heads != pool_key.shape[2] or head_dim != pool_key.shape[3]:
            raise ExecutionError("KV store batch, heads or head dim does not match")
        if positions.shape != (batch,) or positions.dtype != torch.int64:
            raise ExecutionError("KV store positions must be a 1-D batch int64 tensor")
        if positions.device != key.device:
            raise ExecutionError("KV store positions and K/V must share a device")
        return pool_key, pool_value

    def store(self, slot, key, value, positions, *, writer=hip_kv_store) -> "PagedKVCacheState":
        pool_key, pool_value = self._validate_store(slot, key, value, positions)
        if writer is not hip_kv_store:
            raise ExecutionError("a paged KV state stores through its block table only")
        hip_paged_kv_store(pool_key, pool_value, self.block_table, key, value, positions,
                           overflow=self.overflow)
        return self

    def rope_store(self, slot, query, key, value, cosine, sine, positions):
        q_rot, k_rot = hip_rope(query, key, cosine, sine)
        return q_rot, self.store(slot, k_rot, value, positions)

    def rope_store_advance(self, slot, query, key, value, cosine, sine, *, delta):
        if delta <= 0:
            raise ExecutionError("KV advance delta must be positive")
        q_rot, state = self.rope_store(slot, query, key, value, cosine, sine, self.positions(slot))
        return q_rot, state.advance(slot, delta=delta)

    def rope_store_attention(self, slot, query, key, value, cosine, sine, attention_mask, *,
                             groups, scale, softmax_order="online"):
        """One kernel where it takes the case (RoPE, the paged store of the new
        row, the length advance and the paged attention), else the three ops;
        the same result either way."""

        positions = self._check_attention(slot, query, attention_mask, groups)
        self._validate_store(slot, key, value, positions)
        out = positions if self.in_place_lengths else torch.empty_like(positions)
        result = None
        if key.shape[2] == 1:
            result = hip_paged_rope_decode_attention(
                query, key, value, cosine, sine, self.keys[slot], self.values[slot],
                self.block_table, positions, out, _kernel_mask(attention_mask, self.capacity),
                scale=scale, overflow=self.overflow,
                softmax_order=attention_order(softmax_order, attention_mask.shape[-1], query),
                workspace=self.workspace)
        if result is None:
            q_rot, state = self.rope_store_advance(slot, query, key, value, cosine, sine, delta=1)
            return state.decode_attention(slot, q_rot, attention_mask, groups=groups, scale=scale,
                                          softmax_order=softmax_order), state
        lengths = list(self.lengths)
        lengths[slot] = out
        zero = None if self.zero_slots is None else self.zero_slots - {slot}
        return result, replace(self, lengths=tuple(lengths), generation=self.generation + 1,
                               zero_slots=zero)


def _device_workspace(device: torch.device) -> _native.DeviceWorkspace | None:
    return _native.DeviceWorkspace(device) if device.type == "cuda" else None


def mark_zero_mask(mask: torch.Tensor) -> torch.Tensor:
    """Declare ``mask`` an all-zero additive attention mask for as long as it
    lives (its owner never writes it): the HIP decode attention kernels then
    do not read it when it spans the whole capacity.  Adding +0.0 to a score
    changes no result, so the outputs are the same bit for bit; the kernels
    save the mask loads.  The graph decoder's capacity-long mask is one."""

    mask._slc_zero_mask = True
    return mask


def _kernel_mask(mask: torch.Tensor, capacity: int) -> torch.Tensor | None:
    """The mask a HIP decode attention kernel needs: None for a marked zero
    mask over the whole capacity (the kernel's range is then the capacity,
    as it is the mask's), else the mask."""

    if getattr(mask, "_slc_zero_mask", False) and mask.shape[-1] == capacity:
        return None
    return mask


def attention_order(requested: str, mask_len: int, query: torch.Tensor) -> str:
    """The softmax order a decode attention call runs: the requested one, or
    the online order where the exact order does not take the mask length
    (over 4096 tokens at head_dim 64 with bf16/fp16)."""

    if requested == "exact" and mask_len > exact_max_tokens(query.shape[-1], query.dtype):
        return "online"
    return requested


@dataclass
class ExecutionResult:
    outputs: tuple[Any, ...]
    executed_operations: tuple[str, ...]
    symbolic_dimensions: dict[str, int]


class HipExecutor:
    """Executes lowered KernelIR on the gfx950 kernels."""

    def __init__(self, *, strict: bool = True, validate: bool = True) -> None:
        self.strict = strict
        self.validate = validate
        self.lowering_trace: list[dict[str, Any]] = []
        # id(mask) -> (mask, tile classes) for the run in progress.
        self._mask_tiles: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        self._handlers: dict[str, Callable[[list[Any], dict[str, Any]], Any]] = {
            "kernel.hip.rms_norm": self._rms_norm,
            "kernel.hip.linear": self._linear,
            "kernel.hip.rope": self._rope,
            "kernel.hip.prefill_attention": self._prefill_attention,
            "kernel.hip.decode_attention": self._decode_attention,
            "kernel.hip.kv_store": self._kv_store,
            "kernel.hip.kv_prefill_store": self._kv_prefill_store,
            "kernel.hip.embedding": self._embedding,
            "kernel.hip.add": self._add,
            "kernel.hip.swiglu": self._swiglu,
            "kernel.hip.rope_table": self._rope_table,
            "kernel.hip.norm_linear_group": self._norm_linear_group,
            "kernel.hip.norm_linear_swiglu": self._norm_linear_swiglu,
            "kernel.hip.linear_residual": self._linear_residual,
            "kernel.hip.rope_kv_store": self._rope_kv_store,
            "kernel.hip.rope_store_attention": self._rope_store_attention,
            "runtime.kv.init": self._kv_init,
            "runtime.kv.length": self._kv_length,
            "runtime.kv.advance": self._kv_advance,
            "kernel.metadata.view": self._view,
            "kernel.metadata.reshape": self._view,
            "kernel.metadata.transpose": self._transpose,
            "kernel.metadata.unsqueeze": self._unsqueeze,
            "kernel.metadata.getitem": self._getitem,
            "kernel.rocm_compat.rms_norm": self._compat_rms_norm,
            "kernel.rocm_compat.linear": self._compat_linear,
            "kernel.rocm_compat.decode_attention": self._compat_decode_attention,
            "kernel.rocm_compat.prefill_attention": self._compat_prefill_attention,
            "kernel.rocm_compat.rope_table": self._compat_rope_table,
            "kernel.rocm_compat.swiglu": self._compat_swiglu,
        }

    # ------------------------------------------------------------------ run

    def run(self, module: Module, arguments: Sequence[Any], *, function_name: str | None = None) -> ExecutionResult:
        if self.strict:
            # Check the whole graph before any op runs.
            require_full_lowering(module)
        function = select_function(module, function_name)
        if len(arguments) != len(function.block.arguments):
            raise ExecutionError(
                f"@{function.name} takes {len(function.block.arguments)} arguments, got {len(arguments)}"
            )
        environment: dict[str, Any] = {}
        symbols: dict[str, int] = {}
        self._mask_tiles = {}
        for argument, value in zip(function.block.arguments, arguments):
            if self.validate:
                validate_runtime_value(value, argument.type, symbols, context=f"argument {argument.name}")
            environment[argument.name] = value
        trace = []
        for operation in function.block.operations:
            handler = self._handlers.get(operation.name)
            if handler is None:
                raise ExecutionError(f"no gfx950 kernel for operation {operation.name}")
            result = handler([environment[v.name] for v in operation.operands], operation.attributes)
            values = normalize_results(result, len(operation.results), operation.name)
            for ir_value, runtime_value in zip(operation.results, values):
                if self.validate:
                    validate_runtime_value(
                        runtime_value, ir_value.type, symbols,
                        context=f"{operation.name} result {ir_value.name}",
                    )
                environment[ir_value.name] = runtime_value
            trace.append(operation.name)
        outputs = tuple(environment[v.name] for v in function.returns)
        self._mask_tiles = {}
        return ExecutionResult(outputs, tuple(trace), dict(symbols))

    # -------------------------------------------------------------- kernels

    def _rms_norm(self, operands, attributes):
        if len(operands) != 2:
            raise ExecutionError("kernel.hip.rms_norm takes input and weight")
        tensor, weight = operands
        rows = tensor.numel() // tensor.shape[-1]
        choice = choose_variant(attributes.get("lowering_plan"), max(rows, 1))
        self.lowering_trace.append({
            "op": "rms_norm", "backend": "hip", "variant": choice.variant,
            "source": choice.source, "rows": rows, "estimated_us": choice.estimated_us,
        })
        return hip_rms_norm(
            tensor, weight, epsilon=float(attributes["epsilon"]),
            output_dtype=attributes.get("output_dtype"),
            num_warps=waves_per_row(choice.variant) or None,
            round_before_weight=bool(attributes.get("round_before_weight", False)),
        )

    def _linear(self, operands, attributes):
        if len(operands) not in (2, 3):
            raise ExecutionError("kernel.hip.linear takes input, weight and an optional bias")
        bias = operands[2] if len(operands) == 3 else None
        if bool(attributes.get("has_bias")) != (bias is not None):
            raise ExecutionError("kernel.hip.linear has_bias does not match its operands")
        plan = attributes.get("tile_plan")
        tile = "auto"
        if plan is not None:
            rows = operands[0].numel() // max(operands[0].shape[-1], 1)
            choice = choose_variant(plan, max(rows, 1))
            tile = linear_tile(choice.variant)
            self.lowering_trace.append({
                "op": "linear", "backend": "hip", "variant": choice.variant,
                "source": choice.source, "rows": rows, "estimated_us": choice.estimated_us,
            })
        return hip_linear(operands[0], operands[1], bias, tile=tile)

    @staticmethod
    def _rope(operands, attributes):
        if len(operands) != 4:
            raise ExecutionError("kernel.hip.rope takes query, key, cosine and sine")
        if operands[0].shape[-1] != int(attributes["head_dim"]):
            raise ExecutionError("kernel.hip.rope head dim mismatch")
        return hip_rope(*operands)

    def _prefill_attention(self, operands, attributes):
        if len(operands) != 4:
            raise ExecutionError("kernel.hip.prefill_attention takes query, key, value and mask")
        query, key, value, mask = operands
        groups = int(attributes["groups"])
        if query.shape[1] != key.shape[1] * groups:
            raise ExecutionError("kernel.hip.prefill_attention GQA groups do not match")
        tiles = None
        if mask is not None and mask.is_cuda:
            # Every layer applies the function's one mask: classify it once
            # per run (the entry keeps the mask alive, so its id is stable).
            cached = self._mask_tiles.get(id(mask))
            if cached is None or cached[0] is not mask:
                cached = (mask, hip_prefill_mask_tiles(mask))
                self._mask_tiles[id(mask)] = cached
            tiles = cached[1]
        return hip_prefill_attention(
            query, key, value, mask, scale=float(attributes["scale"]),
            causal=attributes.get("causal") is True,
            softmax_order=str(attributes.get("softmax_order", "online")), mask_tiles=tiles,
        )

    def _decode_attention(self, operands, attributes):
        if len(operands) != 3 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("kernel.hip.decode_attention takes state, query and mask")
        state, query, mask = operands
        plan = attributes.get("split_plan")
        split = 0
        if plan is not None:
            choice = choose_variant(plan, max(query.shape[0] * mask.shape[-1], 1))
            split = split_tokens(choice.variant)
            self.lowering_trace.append({
                "op": "decode_attention", "backend": "hip", "variant": choice.variant,
                "source": choice.source, "size": choice.size, "estimated_us": choice.estimated_us,
            })
        order = str(attributes.get("softmax_order", "online"))
        self._trace_order(order, mask, query)
        return state.decode_attention(
            int(attributes.get("slot", 0)), query, mask, groups=int(attributes["groups"]),
            scale=float(attributes["scale"]), softmax_order=order, split_tokens=split,
        )

    def _trace_order(self, requested: str, mask, query) -> None:
        """Record a softmax order the kernel cannot honour: the exact order
        holds each lane's scores in LDS, so masks longer than
        exact_max_tokens run the online order instead."""

        ran = attention_order(requested, mask.shape[-1], query)
        if ran != requested:
            self.lowering_trace.append({
                "op": "decode_attention", "backend": "hip", "softmax_order": ran,
                "requested_softmax_order": requested, "mask_len": int(mask.shape[-1]),
                "reason": f"exact order takes at most {exact_max_tokens(query.shape[-1], query.dtype)} tokens",
            })

    @staticmethod
    def _kv_store(operands, attributes):
        if len(operands) != 4 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("kernel.hip.kv_store takes state, key, value and positions")
        state, key, value, positions = operands
        return state.store(int(attributes.get("slot", 0)), key, value, positions)

    @staticmethod
    def _kv_prefill_store(operands, attributes):
        if len(operands) != 3 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("kernel.hip.kv_prefill_store takes state, key and value")
        state, key, value = operands
        return state.prefill_store(int(attributes.get("slot", 0)), key, value)

    @staticmethod
    def _norm_linear_group(operands, attributes):
        has_bias = list(attributes["has_bias"])
        if len(operands) != 2 + len(has_bias) + sum(has_bias):
            raise ExecutionError("kernel.hip.norm_linear_group operands do not match has_bias")
        tensor, norm_weight = operands[:2]
        weights, biases, i = [], [], 2
        for bias_present in has_bias:
            weights.append(operands[i])
            biases.append(operands[i + 1] if bias_present else None)
            i += 2 if bias_present else 1
        outputs = hip_norm_linear_group(tensor, norm_weight, weights, biases,
                                        epsilon=float(attributes["epsilon"]))
        return outputs[0] if len(outputs) == 1 else tuple(outputs)

    @staticmethod
    def _norm_linear_swiglu(operands, attributes):
        if len(operands) != 4:
            raise ExecutionError("kernel.hip.norm_linear_swiglu takes input, norm, gate and up weights")
        tensor, norm_weight, gate, up = operands
        return hip_norm_linear_swiglu(tensor, norm_weight, gate, up, epsilon=float(attributes["epsilon"]))

    @staticmethod
    def _linear_residual(operands, attributes):
        has_bias = bool(attributes.get("has_bias"))
        if len(operands) != (4 if has_bias else 3):
            raise ExecutionError("kernel.hip.linear_residual takes input, weight, [bias,] residual")
        bias = operands[2] if has_bias else None
        return hip_linear_residual(operands[0], operands[1], bias, operands[-1])

    @staticmethod
    def _rope_kv_store(operands, attributes):
        if len(operands) != 7 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("kernel.hip.rope_kv_store takes state, q, k, v, cos, sin, positions")
        state, query, key, value, cosine, sine, positions = operands
        if query.shape[-1] != int(attributes["head_dim"]):
            raise ExecutionError("kernel.hip.rope_kv_store head dim mismatch")
        slot = int(attributes.get("slot", 0))
        delta = int(attributes.get("advance", 0))
        if delta:
            # positions is this slot's length tensor (the fusion pass checks it).
            return state.rope_store_advance(slot, query, key, value, cosine, sine, delta=delta)
        return state.rope_store(slot, query, key, value, cosine, sine, positions)

    def _rope_store_attention(self, operands, attributes):
        if len(operands) != 8 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError(
                "kernel.hip.rope_store_attention takes state, q, k, v, cos, sin, positions, mask"
            )
        state, query, key, value, cosine, sine, _positions, mask = operands
        if query.shape[-1] != int(attributes["head_dim"]):
            raise ExecutionError("kernel.hip.rope_store_attention head dim mismatch")
        # positions is this slot's length tensor and the advance is one token
        # (the fusion pass checks both).
        order = str(attributes.get("softmax_order", "online"))
        self._trace_order(order, mask, query)
        return state.rope_store_attention(
            int(attributes.get("slot", 0)), query, key, value, cosine, sine, mask,
            groups=int(attributes["groups"]), scale=float(attributes["scale"]),
            softmax_order=order,
        )

    @staticmethod
    def _embedding(operands, attributes):
        ids, table = operands
        return hip_embedding(ids, table)

    @staticmethod
    def _add(operands, attributes):
        return hip_add(*operands)

    @staticmethod
    def _swiglu(operands, attributes):
        return hip_swiglu(*operands)

    @staticmethod
    def _rope_table(operands, attributes):
        positions, inv_freq = operands
        return hip_rope_table(positions, inv_freq, DTYPES[attributes["dtype"]])

    @staticmethod
    def _kv_init(operands, attributes):
        if len(operands) != 1 or not isinstance(operands[0], torch.Tensor):
            raise ExecutionError("runtime.kv.init takes one key template")
        if attributes.get("layout", "contiguous_bshd") == "paged":
            return PagedKVCacheState.empty_from_key_template(
                operands[0], num_layers=int(attributes["num_layers"]),
                capacity=int(attributes["capacity"]), page_tokens=int(attributes["page_tokens"]),
            )
        return PreallocatedKVCacheState.empty_from_key_template(
            operands[0], num_layers=int(attributes["num_layers"]),
            capacity=int(attributes["capacity"]),
        )

    @staticmethod
    def _kv_length(operands, attributes):
        if len(operands) != 1 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("runtime.kv.length takes a KV state")
        return operands[0].positions(int(attributes.get("slot", 0)))

    @staticmethod
    def _kv_advance(operands, attributes):
        if len(operands) != 1 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("runtime.kv.advance takes a KV state")
        return operands[0].advance(int(attributes.get("slot", 0)), delta=int(attributes.get("delta", 1)))

    # -------------------------------------------------------------- metadata

    @staticmethod
    def _view(operands, attributes):
        (tensor,) = operands
        shape = resolve_shape(attributes["shape"], tensor)
        try:
            return tensor.view(shape)
        except RuntimeError as error:
            raise ExecutionError(
                f"metadata view {tuple(tensor.shape)} -> {shape} would need a copy"
            ) from error

    @staticmethod
    def _transpose(operands, attributes):
        (tensor,) = operands
        return tensor.transpose(int(attributes["dim0"]), int(attributes["dim1"]))

    @staticmethod
    def _unsqueeze(operands, attributes):
        (tensor,) = operands
        return tensor.unsqueeze(int(attributes["dim"]))

    @staticmethod
    def _getitem(operands, attributes):
        (value,) = operands
        return value[int(attributes["index"])]

    # --------------------------------------------------------------- compat

    @staticmethod
    def _compat_rms_norm(operands, attributes):
        """PyTorch-ROCm composite with the reference executor's rounding order
        (execution.py:674-692)."""

        _require_gpu(operands, "kernel.rocm_compat.rms_norm")
        tensor, weight = operands
        epsilon = float(attributes["epsilon"])
        variance = tensor.float().pow(2).mean(dim=-1, keepdim=True)
        normalized = tensor.float() * torch.rsqrt(variance + epsilon)
        dtype = DTYPES.get(attributes.get("output_dtype"), tensor.dtype)
        if bool(attributes.get("round_before_weight", False)):
            return weight * normalized.to(dtype)
        return (normalized * weight.float()).to(dtype)

    @staticmethod
    def _compat_linear(operands, attributes):
        """PyTorch's ROCm BLAS GEMM (the reference's kernel.cublas.linear)."""

        _require_gpu(operands, "kernel.rocm_compat.linear")
        bias = operands[2] if len(operands) == 3 else None
        if bool(attributes.get("has_bias")) != (bias is not None):
            raise ExecutionError("kernel.rocm_compat.linear has_bias does not match its operands")
        return F.linear(operands[0], operands[1], bias)

    @staticmethod
    def _compat_decode_attention(operands, attributes):
        """Eager composite of the original graph's GQA attention
        (triton_executor.py:419-463 in the reference)."""

        if len(operands) != 3 or not isinstance(operands[0], PreallocatedKVCacheState):
            raise ExecutionError("kernel.rocm_compat.decode_attention takes state, query and mask")
        state, query, mask = operands
        _require_gpu([query, mask], "kernel.rocm_compat.decode_attention")
        groups = int(attributes["groups"])
        key_buffer, value_buffer, lengths = state._attention_inputs(int(attributes.get("slot", 0)), query, mask, groups)
        sequence = mask.shape[-1]
        key = key_buffer[:, :sequence].permute(0, 2, 1, 3).repeat_interleave(groups, dim=1)
        value = value_buffer[:, :sequence].permute(0, 2, 1, 3).repeat_interleave(groups, dim=1)
        scores = torch.matmul(query, key.transpose(-2, -1)) * float(attributes["scale"])
        scores = scores.float() + mask.float()
        valid = torch.arange(sequence, device=query.device).view(1, 1, 1, sequence) < lengths.view(-1, 1, 1, 1)
        scores = scores.masked_fill(~valid, float("-inf"))
        return torch.matmul(torch.softmax(scores, dim=-1).to(query.dtype), value)

    @staticmethod
    def _compat_prefill_attention(operands, attributes):
        """Eager composite of the original prefill attention (execution.py:707-739)."""

        _require_gpu(operands, "kernel.rocm_compat.prefill_attention")
        query, key, value, mask = operands
        groups = int(attributes["groups"])
        expanded_key = key.repeat_interleave(groups, dim=1)
        expanded_value = value.repeat_interleave(groups, dim=1)
        scores = torch.matmul(query, expanded_key.transpose(-2, -1)) * float(attributes["scale"])
        scores = scores.float() + mask.float()
        if attributes.get("causal") is True:
            tokens = query.shape[2]
            future = torch.triu(torch.ones(tokens, tokens, dtype=torch.bool, device=query.device), diagonal=1)
            scores = scores.masked_fill(future, float("-inf"))
        context = torch.matmul(torch.softmax(scores, dim=-1).to(query.dtype), expanded_value)
        # Same bytes in the [B, T, H, D] layout the head merge views (the eager
        # model makes this copy with .transpose(1, 2).contiguous()).
        return context.transpose(1, 2).contiguous().transpose(1, 2)


    @staticmethod
    def _compat_rope_table(operands, attributes):
        """cos/sin of cat(f, f), f = pos * inv_freq, with PyTorch's kernels
        (qwen2.py:136-149)."""

        _require_gpu(operands, "kernel.rocm_compat.rope_table")
        positions, inv_freq = operands
        freqs = positions.float().unsqueeze(-1) * inv_freq.float().view(1, 1, -1)
        emb = torch.cat((freqs, freqs), dim=-1)
        dtype = DTYPES[attributes["dtype"]]
        return emb.cos().to(dtype), emb.sin().to(dtype)

    @staticmethod
    def _compat_swiglu(operands, attributes):
        """silu(gate) * up with PyTorch's SiLU (qwen2.py:253-256)."""

        _require_gpu(operands, "kernel.rocm_compat.swiglu")
        return F.silu(operands[0]) * operands[1]


def _require_gpu(operands: Sequence[Any], what: str) -> None:
    tensors = [o for o in operands if isinstance(o, torch.Tensor)]
    if not tensors or not all(t.is_cuda for t in tensors):
        raise ExecutionError(f"{what}: every tensor must be on the GPU")


def resolve_shape(spec: Sequence[Any], tensor: torch.Tensor) -> list[int]:
    """View shapes: ints, -1, or {"dim": i} for the input's size at axis i."""

    shape = []
    for item in spec:
        if isinstance(item, dict) and "dim" in item:
            shape.append(int(tensor.shape[int(item["dim"])]))
        else:
            shape.append(int(item))
    return shape


def select_function(module: Module, function_name: str | None) -> Function:
    if function_name is None:
        if len(module.functions) != 1:
            raise ExecutionError("the module has several functions; pass function_name")
        return module.functions[0]
    for function in module.functions:
        if function.name == function_name:
            return function
    raise ExecutionError(f"no function @{function_name}")


def normalize_results(result: Any, expected: int, name: str) -> tuple[Any, ...]:
    if expected == 0:
        if result is not None:
            raise ExecutionError(f"{name} must not produce a result")
        return ()
    if expected == 1:
        return (result,)
    if not isinstance(result, (tuple, list)) or len(result) != expected:
        raise ExecutionError(f"{name} must produce {expected} results")
    return tuple(result)


def validate_runtime_value(value: Any, type_: IRType, symbols: dict[str, int], *, context: str) -> None:
    """Type / shape / device / symbol guard (execution.py:1094-1157)."""

    if isinstance(type_, UnknownType):
        return
    if isinstance(type_, TensorType):
        if not isinstance(value, torch.Tensor):
            raise ExecutionError(f"{context} must be a tensor")
        expected = DTYPES.get(type_.dtype)
        if expected is not None and value.dtype != expected:
            raise ExecutionError(f"{context} dtype must be {expected}, got {value.dtype}")
        if str(value.device) != type_.device:
            raise ExecutionError(f"{context} device must be {type_.device}, got {value.device}")
        if value.ndim != len(type_.shape):
            raise ExecutionError(f"{context} rank must be {len(type_.shape)}, got {value.ndim}")
        for index, (actual, dimension) in enumerate(zip(value.shape, type_.shape)):
            if isinstance(dimension, StaticDim):
                if actual != dimension.value:
                    raise ExecutionError(f"{context} dim {index} must be {dimension.value}, got {actual}")
            elif isinstance(dimension, SymbolicDim):
                _bind_symbol(dimension, int(actual), symbols, context, index)
        return
    if isinstance(type_, KVStateType):
        _validate_kv_state(value, type_, context)
        return
    if isinstance(type_, TupleType):
        if not isinstance(value, (tuple, list)) or len(value) != len(type_.elements):
            raise ExecutionError(f"{context} must be a tuple of {len(type_.elements)}")
        for index, (item, item_type) in enumerate(zip(value, type_.elements)):
            validate_runtime_value(item, item_type, symbols, context=f"{context}[{index}]")
        return
    if isinstance(type_, ScalarType):
        if type_.dtype in {"index", "symint"} and not isinstance(value, int):
            raise ExecutionError(f"{context} must be an integer scalar")
        return
    raise ExecutionError(f"{context} has a type that cannot execute: {type_}")


def _validate_kv_state(value: Any, type_: KVStateType, context: str) -> None:
    if not isinstance(value, PreallocatedKVCacheState):
        raise ExecutionError(f"{context} must be a preallocated KV runtime state")
    paged = isinstance(value, PagedKVCacheState)
    if type_.layout == "paged":
        if not paged:
            raise ExecutionError(f"{context} must be a paged KV state")
        if type_.page_tokens is not None and value.page_tokens != type_.page_tokens:
            raise ExecutionError(f"{context} page_tokens must be {type_.page_tokens}, got {value.page_tokens}")
    elif type_.layout == "contiguous_bshd":
        if paged:
            raise ExecutionError(f"{context} must be a contiguous_bshd KV state, got a paged one")
    else:
        raise ExecutionError(f"{context}: layout {type_.layout} is not supported by the runtime")
    if type_.capacity is not None and value.capacity != type_.capacity:
        raise ExecutionError(f"{context} capacity must be {type_.capacity}, got {value.capacity}")
    if len(value.keys) != type_.num_layers:
        raise ExecutionError(f"{context} must hold {type_.num_layers} layer slots")
    expected = DTYPES.get(type_.dtype)
    for slot, key in enumerate(value.keys):
        if key.shape[2] != type_.num_kv_heads or key.shape[3] != type_.head_dim:
            raise ExecutionError(f"{context} slot {slot} heads/head dim do not match")
        if expected is not None and key.dtype != expected:
            raise ExecutionError(f"{context} slot {slot} dtype must be {expected}")


def _bind_symbol(dimension: SymbolicDim, actual: int, symbols: dict[str, int], context: str, index: int) -> None:
    existing = symbols.get(dimension.name)
    if existing is not None and existing != actual:
        raise ExecutionError(
            f"{context} dim {index} breaks symbol {dimension.name}: bound to {existing}, got {actual}"
        )
    lower, upper = _parse_bounds(dimension.bounds)
    if lower is not None and actual < lower:
        raise ExecutionError(f"{context} dim {index}: {dimension.name}={actual} below {lower}")
    if upper is not None and actual > upper:
        raise ExecutionError(f"{context} dim {index}: {dimension.name}={actual} above {upper}")
    symbols[dimension.name] = actual


def _parse_bounds(bounds: str | None) -> tuple[int | None, int | None]:
    if not bounds:
        return None, None
    match = re.fullmatch(r"VR\[(-?\d+),\s*(-?\d+|int_oo)\]", bounds)
    if match is None:
        return None, None
    return int(match.group(1)), None if match.group(2) == "int_oo" else int(match.group(2))
