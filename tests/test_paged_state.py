"""Host logic of the paged KV state (CPU tensors; no kernel runs): the
construction checks, the page order of a fresh state, and the gather / read
that eager composites and inspection use."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kernels as ref
from stateful_llm_compiler_hip.execution import ExecutionError, PagedKVCacheState


def _state(batch=2, pages=4, page_tokens=16, heads=2, dim=8, num_pages=None, table=None, layers=1):
    num_pages = batch * pages if num_pages is None else num_pages
    keys = tuple(torch.randn(num_pages, page_tokens, heads, dim) for _ in range(layers))
    values = tuple(torch.randn(num_pages, page_tokens, heads, dim) for _ in range(layers))
    lengths = tuple(torch.zeros(batch, dtype=torch.int64) for _ in range(layers))
    if table is None:
        table = torch.arange(batch * pages, dtype=torch.int32).view(batch, pages)
    return PagedKVCacheState(keys, values, lengths, pages * page_tokens, block_table=table,
                             page_tokens=page_tokens)


@pytest.mark.parametrize("kwargs,needle", [
    ({"page_tokens": 24}, "power of two"),
    ({"page_tokens": 8}, "power of two"),
    ({"table": torch.zeros(2, 3, dtype=torch.int32)}, "capacity / page_tokens"),
    ({"table": torch.zeros(2, 4, dtype=torch.int64)}, "int32"),
    ({"table": torch.tensor([[0, 1, 2, 3], [4, 5, 6, 8]], dtype=torch.int32)}, r"\[0, 8\)"),
    ({"table": torch.tensor([[0, 1, 2, 3], [4, -1, 6, 7]], dtype=torch.int32)}, "pool page indices"),
])
def test_paged_state_rejects_bad_geometry(kwargs, needle):
    with pytest.raises(ExecutionError, match=needle):
        _state(**kwargs)


def test_paged_state_rejects_mismatched_pools_and_lengths():
    state = _state()
    with pytest.raises(ExecutionError):
        PagedKVCacheState(state.keys, (torch.randn(8, 16, 2, 4),), state.lengths, state.capacity,
                          block_table=state.block_table, page_tokens=16)
    with pytest.raises(ExecutionError):
        PagedKVCacheState(state.keys, state.values, (torch.zeros(3, dtype=torch.int64),),
                          state.capacity, block_table=state.block_table, page_tokens=16)


def test_gather_matches_the_oracle_and_read_slices_the_prefix():
    g = torch.Generator().manual_seed(3)
    table = torch.randperm(8, generator=g).view(2, 4).to(torch.int32)
    state = _state(table=table)
    key, value = state.gather(0)
    assert torch.equal(key, torch.from_numpy(ref.gather_pages(state.keys[0].numpy(), table.numpy())))
    assert torch.equal(value, torch.from_numpy(ref.gather_pages(state.values[0].numpy(), table.numpy())))
    lengths = torch.tensor([5, 40], dtype=torch.int64)
    from dataclasses import replace
    state = replace(state, lengths=(lengths,))
    rk, rv = state.read(0)
    assert rk.shape == (2, 2, 40, 8)
    assert torch.equal(rk, key[:, :40].transpose(1, 2)) and torch.equal(rv, value[:, :40].transpose(1, 2))


def test_fresh_state_scatters_every_sequence_over_the_pool():
    template = torch.zeros(3, 2, 1, 8, dtype=torch.bfloat16)
    state = PagedKVCacheState.empty_from_key_template(template, num_layers=2, capacity=64, page_tokens=16)
    table = state.block_table.numpy()
    assert table.shape == (3, 4)
    assert sorted(table.ravel().tolist()) == list(range(12))  # every page owned once
    assert np.array_equal(table[:, 1] - table[:, 0], np.full(3, 3))  # page j of b = j * B + b
    assert state.keys[0].shape == (12, 16, 2, 8) and len(state.keys) == 2
    assert state.zero_slots == frozenset({0, 1})
