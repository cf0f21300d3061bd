"""Seeded synthetic inputs for the BASELINE configurations (host numpy arrays).

All randomness comes from ``numpy.random.default_rng(seed)`` (PCG64), so the GPU path and
the CPU oracle see bit-identical inputs.  Layouts follow include/ferrisinfer_kernel.h.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class PagedDecodeWorkload:
    """Config C2: standalone paged decode attention over a shared block pool."""

    num_seqs: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    context_lens: np.ndarray   # int32 [B]
    block_tables: np.ndarray   # int32 [B, max_blocks]
    q: np.ndarray              # f32 [B, Hq, D]
    k_pool: np.ndarray         # f32 [num_blocks, Hkv, bs, D]  (device layout)
    v_pool: np.ndarray
    scale: float

    @property
    def max_context_len(self) -> int:
        return int(self.context_lens.max())

    def pages_reference_layout(self, pool: np.ndarray) -> np.ndarray:
        """[num_blocks, Hkv, bs, D] -> the reference page layout [num_blocks, bs, Hkv, D]
        (runtime/paged_kv.rs:141-150)."""
        return np.ascontiguousarray(pool.transpose(0, 2, 1, 3))

    def algorithmic_bytes(self, kv_bytes: int = 4) -> int:
        """Bytes one launch must move: every context K/V row once, q in, out back, block
        table entries and context lengths."""
        L = self.context_lens.astype(np.int64)
        kv = int(L.sum()) * self.num_kv_heads * self.head_dim * 2 * kv_bytes
        qo = self.num_seqs * self.num_q_heads * self.head_dim * (4 + 4)
        bt = int(((L + self.block_size - 1) // self.block_size).sum()) * 4
        return kv + qo + bt + self.num_seqs * 4


def paged_decode_c2(seed: int = 0, num_seqs: int = 64, min_len: int = 128, max_len: int = 2048,
                    num_q_heads: int = 32, num_kv_heads: int = 8, head_dim: int = 128,
                    block_size: int = 16, num_blocks: int = 8192,
                    fill_unused_blocks: bool = False) -> PagedDecodeWorkload:
    """C2: lengths ~ U[min_len, max_len]; block ids are the first sum(ceil(L/bs)) entries of a
    seeded permutation of the pool, handed to the sequences in order; Q/K/V ~ N(0, 1);
    scale 1/sqrt(D).  Unused pool blocks are zero unless ``fill_unused_blocks``."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(min_len, max_len + 1, size=num_seqs).astype(np.int32)
    nblk = (lens + block_size - 1) // block_size
    total = int(nblk.sum())
    if total > num_blocks:
        raise ValueError(f"workload needs {total} blocks, pool has {num_blocks}")
    perm = rng.permutation(num_blocks).astype(np.int32)
    max_blocks = int(nblk.max())
    tables = np.zeros((num_seqs, max_blocks), np.int32)
    cursor = 0
    for i, n in enumerate(nblk):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    q = rng.standard_normal((num_seqs, num_q_heads, head_dim), dtype=np.float32)
    shape = (num_blocks, num_kv_heads, block_size, head_dim)
    k_pool = np.zeros(shape, np.float32)
    v_pool = np.zeros(shape, np.float32)
    used = perm[:total] if not fill_unused_blocks else perm
    k_pool[used] = rng.standard_normal((used.size,) + shape[1:], dtype=np.float32)
    v_pool[used] = rng.standard_normal((used.size,) + shape[1:], dtype=np.float32)
    return PagedDecodeWorkload(num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                               num_blocks, lens, tables, q, k_pool, v_pool,
                               float(1.0 / np.sqrt(np.float32(head_dim))))
