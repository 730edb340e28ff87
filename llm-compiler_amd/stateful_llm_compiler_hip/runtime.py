"""Stateful Qwen2 serving runtime over the compiled KernelIR.

Compiles the prefill and decode functions once (strict full lowering), runs
them through ``HipExecutor``, and can capture one greedy decode step -- the
whole 24-layer KernelIR function plus the next-token argmax -- as a HIP graph.
The KV buffers never move and the lengths advance in place, so replaying the
graph is a decode step with no Python per-op dispatch.  This is the
"stable buffer addresses" property the reference's bufferization establishes
(docs/kv-bufferization.md:160-161) put to use.
"""

from __future__ import annotations

from pathlib import Path

from dataclasses import replace
from typing import Any

import torch

from ._native import DeviceWorkspace
from .backends import hip_argmax
from .compiler import CompileOptions, compile_module
from .execution import HipExecutor, PreallocatedKVCacheState, mark_zero_mask
from .qwen2 import Qwen2Config, build_decode_module, build_prefill_module, weight_arguments


class Qwen2Runtime:
    def __init__(
        self,
        config: Qwen2Config,
        weights: dict[str, torch.Tensor],
        *,
        capacity: int,
        dtype: torch.dtype = torch.bfloat16,
        device: str = "cuda:0",
        numerical_mode: str = "fast",
        mask_dtype: str = "f32",
        validate: bool = True,
        fuse: bool = True,
        attention_softmax: str = "exact",
        linear_backend: str | None = None,
        profile: str | Path | None = None,
        page_tokens: int | None = None,
    ) -> None:
        """``page_tokens``: run on the paged KV layout (page pools + block
        table, ``page_tokens`` tokens a page) instead of contiguous buffers."""
        self.config = config
        self.capacity = capacity
        self.dtype = dtype
        self.device = torch.device(device)
        options = CompileOptions(numerical_mode=numerical_mode, require_full_lowering=True, fuse=fuse,
                                 attention_softmax=attention_softmax, linear_backend=linear_backend,
                                 rmsnorm_profile=profile)
        self.prefill_result = compile_module(
            build_prefill_module(config, capacity=capacity, dtype=dtype, device=device,
                                 mask_dtype=mask_dtype, page_tokens=page_tokens), options)
        self.decode_result = compile_module(
            build_decode_module(config, capacity=capacity, dtype=dtype, device=device,
                                page_tokens=page_tokens), options)
        self.executor = HipExecutor(strict=True, validate=validate)
        self.weight_args = weight_arguments(config, weights)

    def prefill(self, input_ids: torch.Tensor, attention_mask: torch.Tensor,
                position_ids: torch.Tensor) -> tuple[torch.Tensor, PreallocatedKVCacheState]:
        result = self.executor.run(self.prefill_result.module,
                                   [input_ids, attention_mask, position_ids] + self.weight_args)
        return result.outputs

    def decode(self, input_ids: torch.Tensor, attention_mask: torch.Tensor,
               state: PreallocatedKVCacheState) -> tuple[torch.Tensor, PreallocatedKVCacheState]:
        result = self.executor.run(self.decode_result.module,
                                   [input_ids, attention_mask, state] + self.weight_args)
        return result.outputs

    def graph_decoder(self, state: PreallocatedKVCacheState, first_tokens: torch.Tensor) -> "GraphDecoder":
        return GraphDecoder(self, state, first_tokens)


class GraphDecoder:
    """One greedy decode step captured as a HIP graph.

    ``step()`` replays: embed the current tokens, run every layer against the
    KV state (store at the current lengths, advance the lengths in place,
    decode attention over the capacity-long zero mask), LM head, argmax back
    into the token buffer.  ``tokens`` and ``logits`` are fixed tensors that
    the caller may read after each step.
    """

    def __init__(self, runtime: Qwen2Runtime, state: PreallocatedKVCacheState, first_tokens: torch.Tensor) -> None:
        self.runtime = runtime
        batch = first_tokens.shape[0]
        self.tokens = first_tokens.reshape(batch, 1).to(torch.int64).contiguous().clone()
        # All zeros for the decoder's life (never written), so the attention
        # kernels skip it.
        self.mask = mark_zero_mask(
            torch.zeros(batch, 1, 1, runtime.capacity, dtype=runtime.dtype, device=runtime.device))
        # The decoder's own scratch (arrival counters, partials): graphs of two
        # decoders may replay concurrently on different streams.
        self.workspace = DeviceWorkspace(runtime.device)
        self.state = replace(state, in_place_lengths=True, workspace=self.workspace)
        self._warm_up(state)
        self.graph = torch.cuda.CUDAGraph()
        self._stream = torch.cuda.Stream(device=runtime.device)
        self._stream.wait_stream(torch.cuda.current_stream(runtime.device))
        with torch.cuda.stream(self._stream):
            with torch.cuda.graph(self.graph, stream=self._stream):
                logits, self.final_state = runtime.decode(self.tokens, self.mask, self.state)
                self.logits = logits
                hip_argmax(logits[:, -1], out=self.tokens.view(-1), workspace=self.workspace)
        torch.cuda.current_stream(runtime.device).wait_stream(self._stream)

    def _warm_up(self, state: PreallocatedKVCacheState) -> None:
        """Run one step on a scratch copy of the state so every kernel and
        allocation exists before capture."""

        scratch = replace(
            state, keys=tuple(k.clone() for k in state.keys), values=tuple(v.clone() for v in state.values),
            lengths=tuple(n.clone() for n in state.lengths),
            overflow=torch.zeros(1, dtype=torch.int32, device=self.runtime.device),
            in_place_lengths=True, workspace=self.workspace, zero_slots=None,
        )
        logits, _ = self.runtime.decode(self.tokens.clone(), self.mask, scratch)
        hip_argmax(logits[:, -1], workspace=self.workspace)
        torch.cuda.synchronize(self.runtime.device)

    def step(self) -> None:
        self.graph.replay()
