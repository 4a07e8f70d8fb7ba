"""KV cache of the decode path, held in one region of the resident arena.

Storage is a single bf16 tensor ``[num_layers, 2, n_kv, capacity, head_dim]``
-- for each layer its key block, then its value block -- normally the
arena's ``kv_cache`` entry, so the cache lives in the same allocation as the
weights.  Each block is a contiguous ``[n_kv, capacity, head_dim]`` tensor,
the form the decode attention kernel addresses: the kernel writes a token's
key and value row itself and the cache only moves the layer's cursor.

The decode dispatch reads three things from a cache (the static-cache
interface of the reference runtime, src/leanstack/runtime/kv_cache.py:207-266):
``layer_seq_lens[layer]``, ``layer_tensors(layer)`` and ``advance(layer, n)``.
Rows produced by the torch glue (prefill and verify blocks) enter through
``write_rows``; a speculative verify that rejects drafted tokens rolls the
cursors back with ``mark`` / ``rewind``
(experiments/models/qwen_explicit_runtime_loop.py:822-847).  Batch 1 only:
the decode kernels serve one sequence.
"""

from __future__ import annotations

import torch


class ArenaKVCache:
    """Per-layer key/value blocks over one storage tensor, with a row cursor per layer.

    storage: None to allocate zero-filled blocks on `device`, or an existing
    ``[L, 2, n_kv, capacity, d]`` tensor (a ``[L, 2, 1, n_kv, capacity, d]``
    arena entry with its batch axis of 1 is accepted too) that the cache
    then works in place."""

    def __init__(self, num_layers: int, num_key_value_heads: int, head_dim: int, capacity: int, *,
                 storage: torch.Tensor | None = None, device: torch.device | str = "cpu",
                 dtype: torch.dtype = torch.bfloat16) -> None:
        dims = (num_layers, num_key_value_heads, head_dim, capacity)
        if min(dims) < 1:
            raise ValueError(f"cache dimensions must all be >= 1 (layers, kv heads, head_dim, capacity) = {dims}")
        shape = (num_layers, 2, num_key_value_heads, capacity, head_dim)
        if storage is None:
            storage = torch.zeros(shape, device=device, dtype=dtype)
        else:
            if storage.dim() == 6 and storage.shape[2] == 1:
                storage = storage[:, :, 0]
            if tuple(storage.shape) != shape or not storage.is_contiguous():
                raise ValueError(f"cache storage must be a contiguous {list(shape)} tensor "
                                 f"(layers, key|value, kv heads, rows, head_dim); got {list(storage.shape)}")
        self.storage = storage
        self.capacity = capacity
        self.layer_seq_lens = [0] * num_layers

    @classmethod
    def from_arena(cls, arena, num_key_value_heads: int, head_dim: int) -> "ArenaKVCache":
        """The cache over a resident arena's `kv_cache` entry."""
        region = arena.view("kv_cache")
        if region.dim() != 6 or region.shape[2] != 1:
            raise ValueError(f"the arena's kv_cache entry {list(region.shape)} is not a batch-1 cache")
        return cls(region.shape[0], num_key_value_heads, head_dim, region.shape[4], storage=region)

    # -- what the decode dispatch reads --------------------------------------

    def layer_tensors(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The layer's whole key and value blocks, [n_kv, capacity, d] each."""
        return self.storage[layer, 0], self.storage[layer, 1]

    def advance(self, layer: int, rows: int) -> None:
        """Count `rows` rows written after the layer's cursor (by the decode
        attention kernel or write_rows)."""
        new = self.layer_seq_lens[layer] + rows
        if rows < 0 or new > self.capacity:
            raise ValueError(f"layer {layer}: cursor {self.layer_seq_lens[layer]} + {rows} rows does not fit "
                             f"the {self.capacity}-row cache")
        self.layer_seq_lens[layer] = new

    # -- the torch glue's side -----------------------------------------------

    @property
    def key_cache(self) -> torch.Tensor:
        """All key blocks with a batch axis of 1, [L, 1, n_kv, capacity, d]."""
        return self.storage[:, 0].unsqueeze(1)

    @property
    def value_cache(self) -> torch.Tensor:
        return self.storage[:, 1].unsqueeze(1)

    @property
    def max_layer_seq_len(self) -> int:
        return max(self.layer_seq_lens)

    def rows(self, layer: int) -> int:
        return self.layer_seq_lens[layer]

    def write_rows(self, layer: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Copy key / value rows ([n_kv, T, d], or [1, n_kv, T, d]) to the
        layer's cursor and move it past them.  Nothing moves if they do not
        fit."""
        k_block, v_block = self.layer_tensors(layer)
        keys = keys[0] if keys.dim() == 4 and keys.shape[0] == 1 else keys
        values = values[0] if values.dim() == 4 and values.shape[0] == 1 else values
        if keys.shape != values.shape or keys.dim() != 3 or keys.shape[0] != k_block.shape[0] \
                or keys.shape[2] != k_block.shape[2]:
            raise ValueError(f"keys {list(keys.shape)} and values {list(values.shape)} must both be "
                             f"[{k_block.shape[0]}, rows, {k_block.shape[2]}]")
        start = self.layer_seq_lens[layer]
        self.advance(layer, keys.shape[1])
        k_block[:, start : start + keys.shape[1]].copy_(keys)
        v_block[:, start : start + keys.shape[1]].copy_(values)

    def attended(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The layer's written rows as [1, n_kv, rows, d] views (what the
        torch glue attends over)."""
        k_block, v_block = self.layer_tensors(layer)
        n = self.layer_seq_lens[layer]
        return k_block[None, :, :n], v_block[None, :, :n]

    def mark(self) -> tuple[int, ...]:
        """The cursors now, for rewind()."""
        return tuple(self.layer_seq_lens)

    def rewind(self, mark: tuple[int, ...]) -> None:
        """Move the cursors back to `mark`: rows written since are dropped
        (and overwritten by the next writes)."""
        if len(mark) != len(self.layer_seq_lens) or any(m > n or m < 0 for m, n in zip(mark, self.layer_seq_lens)):
            raise ValueError(f"mark {mark} is not an earlier state of the cursors {tuple(self.layer_seq_lens)}")
        self.layer_seq_lens = list(mark)
