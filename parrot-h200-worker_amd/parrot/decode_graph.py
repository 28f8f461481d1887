"""HIP-graph replay of cached decode steps.

A decode step of the HIP backend has static shapes: the attention kernels
read the generation position from ``GenerationState.position_device`` and the
step advances it on the device.  ``DecodeGraph`` captures one
``Parrot.decode_step`` for a given state once and replays it per token, which
removes the host launch cost of the ~30 kernels per layer (the reference
reaches the same end on Apple GPUs with fused decode kernels,
parrot/metal_moe.py:182-221 and parrot/model.py:832-925).
"""
from __future__ import annotations

import torch
from torch import Tensor

from .model import GenerationState, Parrot


class DecodeGraph:
    """Captured ``decode_step`` for one generation state.

    ``step(ids)`` appends one token per sequence (ids ``[batch, 1]``) and
    returns the next greedy tokens ``[batch, 1]`` (or the logits
    ``[batch, 1, vocab]`` with ``logits=True``), exactly as
    ``model.decode_next`` / ``model.decode_step`` would on the same state.
    The returned tensor is the graph's static output, overwritten by the next
    step; for greedy tokens it is the graph's input buffer itself (the step's
    last launch writes the tokens there), so feeding it back to ``step``
    costs no copy.  Both run in inference mode, as ``prefill`` /
    ``decode_step`` do.  The state must stay with this object: eager decode
    steps on it in between are allowed (they advance both positions
    consistently).
    """

    @torch.inference_mode()
    def __init__(self, model: Parrot, state: GenerationState, logits: bool = False):
        if state.position_device is None:
            raise RuntimeError("DecodeGraph needs a generation state from a HIP-backend prefill")
        if model.training:
            raise RuntimeError("DecodeGraph requires model.eval()")
        self.model, self.state, self.logits = model, state, logits
        device = state.position_device.device
        self.ids = torch.zeros((state.batch_size, 1), dtype=torch.long, device=device)
        start = state.position
        if start >= model.config.max_seq_len:
            raise ValueError("Generation state has reached max_seq_len")
        # One eager step on a side stream fills every lazily built cache
        # (packed weights, absorbed maps, RoPE tables, scratch buffers);
        # its cache row at `start` is rewritten by the first real step.
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            self._run()
        torch.cuda.current_stream(device).wait_stream(side)
        self._rewind(start)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = self._run()
        self._rewind(start)

    def _run(self) -> Tensor:
        if self.logits:
            out, _ = self.model.decode_step(self.ids, self.state)
        else:
            # The tokens land in the input buffer, read by the next replay's
            # first launch (the embedding gather), after this step's reads.
            out, _ = self.model.decode_step(self.ids, self.state, _next_token_only=True,
                                            _out=self.ids)
        return out

    def _rewind(self, position: int) -> None:
        self.state.position = position
        self.state.position_device.fill_(position)

    @torch.inference_mode()
    def step(self, input_ids: Tensor) -> Tensor:
        if input_ids.shape != self.ids.shape:
            raise ValueError("decode input must be [cached batch, 1]")
        if self.state.position >= self.model.config.max_seq_len:
            raise ValueError("Generation state has reached max_seq_len")
        if input_ids.data_ptr() != self.ids.data_ptr():
            self.ids.copy_(input_ids)
        self.graph.replay()
        self.state.position += 1
        return self.out
