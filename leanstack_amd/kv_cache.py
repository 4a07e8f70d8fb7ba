"""Static KV cache with the reference's interface (src/leanstack/runtime/kv_cache.py:8-35, :207-330).

`StaticKVBlockManager` keeps key and value tensors of shape
[num_layers, batch_size, num_key_value_heads, max_seq_len, head_dim] and one
sequence length per layer, as the reference's static manager does.  They may
be views of the resident arena's `kv_cache` entry ([L, 2, B, n_kv, S, d]),
so the cache lives in the same allocation as the weights.  The decode
attention kernel (kernels.decode_attention) writes a token's k and v itself;
`advance` then moves the layer's cursor, as `append` does after its copy.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class KVPageLayout:
    """Geometry of the cache (src/leanstack/runtime/kv_cache.py:8-35)."""

    num_layers: int
    num_key_value_heads: int
    head_dim: int
    page_size: int
    max_seq_len: int
    batch_size: int
    dtype: torch.dtype
    device: torch.device

    def __post_init__(self) -> None:
        if self.page_size <= 0:
            raise ValueError("page_size must be positive")
        if self.max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive")
        if self.batch_size <= 0:
            raise ValueError("batch_size must be positive")

    @property
    def num_pages(self) -> int:
        return (self.max_seq_len + self.page_size - 1) // self.page_size

    def pages_for_tokens(self, token_count: int) -> int:
        if token_count <= 0:
            return 0
        return (token_count + self.page_size - 1) // self.page_size


@dataclass(frozen=True)
class StaticKVCursorSnapshot:
    layer_seq_lens: tuple[int, ...]
    max_layer_seq_len: int


class StaticKVBlockManager:
    """Static KV cache (src/leanstack/runtime/kv_cache.py:207-330).

    storage: None (zero-filled tensors of the layout's shape are allocated),
    or a [num_layers, 2, batch_size, n_kv, max_seq_len, head_dim] tensor whose
    [:, 0] / [:, 1] halves become the key / value caches (the arena's
    `kv_cache` entry)."""

    def __init__(self, layout: KVPageLayout, storage: torch.Tensor | None = None):
        self.layout = layout
        shape = (layout.num_layers, layout.batch_size, layout.num_key_value_heads, layout.max_seq_len,
                 layout.head_dim)
        if storage is None:
            self.key_cache = torch.zeros(shape, device=layout.device, dtype=layout.dtype)
            self.value_cache = torch.zeros(shape, device=layout.device, dtype=layout.dtype)
        else:
            expect = (layout.num_layers, 2) + shape[1:]
            if tuple(storage.shape) != expect or storage.dtype != layout.dtype:
                raise ValueError(f"storage must be {layout.dtype} {expect}, got {storage.dtype} {tuple(storage.shape)}")
            self.key_cache = storage[:, 0]
            self.value_cache = storage[:, 1]
        self.layer_seq_lens = [0 for _ in range(layout.num_layers)]
        self.max_layer_seq_len = 0

    def append(self, layer_idx: int, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Copy [B, n_kv, T, d] key / value states after the layer's cached rows."""
        if key_states.shape != value_states.shape:
            raise ValueError("key/value states must have the same shape")
        batch_size, num_heads, token_count, head_dim = key_states.shape
        if batch_size != self.layout.batch_size:
            raise ValueError(f"expected batch_size={self.layout.batch_size}, got {batch_size}")
        if num_heads != self.layout.num_key_value_heads:
            raise ValueError(f"expected num_key_value_heads={self.layout.num_key_value_heads}, got {num_heads}")
        if head_dim != self.layout.head_dim:
            raise ValueError(f"expected head_dim={self.layout.head_dim}, got {head_dim}")
        start = self.layer_seq_lens[layer_idx]
        end = start + token_count
        if end > self.layout.max_seq_len:
            raise ValueError(
                f"cache overflow for layer {layer_idx}: requested {end} tokens with max_seq_len={self.layout.max_seq_len}"
            )
        self.key_cache[layer_idx, :, :, start:end, :].copy_(key_states)
        self.value_cache[layer_idx, :, :, start:end, :].copy_(value_states)
        self.advance(layer_idx, token_count)

    def advance(self, layer_idx: int, token_count: int) -> None:
        """Count `token_count` rows written after the layer's cached ones."""
        end = self.layer_seq_lens[layer_idx] + token_count
        if end > self.layout.max_seq_len:
            raise ValueError(f"cache overflow for layer {layer_idx}: {end} > max_seq_len={self.layout.max_seq_len}")
        self.layer_seq_lens[layer_idx] = end
        self.max_layer_seq_len = max(self.max_layer_seq_len, end)

    def append_and_get(self, layer_idx: int, key_states: torch.Tensor,
                       value_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        self.append(layer_idx, key_states, value_states)
        return self.get(layer_idx)

    def get(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        seq_len = self.layer_seq_lens[layer_idx]
        return self.key_cache[layer_idx, :, :, :seq_len, :], self.value_cache[layer_idx, :, :, :seq_len, :]

    def layer_tensors(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The layer's whole [n_kv, max_seq_len, head_dim] key / value caches
        (batch 1), as the decode attention kernel addresses them."""
        if self.layout.batch_size != 1:
            raise ValueError("the decode attention kernel serves batch 1")
        return self.key_cache[layer_idx, 0], self.value_cache[layer_idx, 0]

    def get_layer_seq_length(self, layer_idx: int) -> int:
        return self.layer_seq_lens[layer_idx]

    def get_seq_length(self) -> int:
        return self.max_layer_seq_len

    def page_table(self, layer_idx: int) -> tuple[int, ...]:
        return tuple(range(self.layout.pages_for_tokens(self.get_layer_seq_length(layer_idx))))

    def snapshot_cursor(self) -> StaticKVCursorSnapshot:
        return StaticKVCursorSnapshot(tuple(int(n) for n in self.layer_seq_lens), int(self.max_layer_seq_len))

    def restore_cursor(self, snapshot: StaticKVCursorSnapshot) -> None:
        self.layer_seq_lens = list(snapshot.layer_seq_lens)
        self.max_layer_seq_len = int(snapshot.max_layer_seq_len)
