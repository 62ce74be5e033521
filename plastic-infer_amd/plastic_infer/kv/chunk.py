"""Chunk keys: deterministic chained SHA-256 over token ids (prefix reuse of KV chunks).

Key format kept identical to the reference (src/plastic_infer/kv/chunk.py:48-149) so that keys
computed by either implementation address the same chunks:
    h_0      = sha256(b"plastic-infer-kv-v1")
    c_i      = sha256(token ids of chunk i, each as 4-byte little-endian unsigned)
    h_{i+1}  = sha256(h_i || c_i)
ChunkKey i = (prefix_key = h_i, cumulative_key = h_{i+1}); lookups use the cumulative key.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

DEFAULT_CHUNK_SIZE: int = 256
_INITIAL_SALT = b"plastic-infer-kv-v1"


@dataclass(frozen=True)
class ChunkKey:
    prefix_key: bytes
    cumulative_key: bytes

    def __repr__(self) -> str:
        return f"ChunkKey({self.cumulative_key.hex()[:16]})"

    @property
    def full_key(self) -> bytes:
        return self.cumulative_key


def _compute(tokens: list[int], chunk_size: int, salt: bytes) -> tuple[list[ChunkKey], bytes]:
    if len(tokens) % chunk_size:
        raise ValueError(f"token count {len(tokens)} not aligned to chunk_size {chunk_size}")
    # One little-endian uint32 buffer for all tokens; each chunk hashes one slice of it.
    raw = np.asarray(tokens, dtype=np.int64).astype("<u4", copy=False).tobytes()
    step = 4 * chunk_size
    running = hashlib.sha256(salt).digest()
    keys: list[ChunkKey] = []
    for off in range(0, len(raw), step):
        content = hashlib.sha256(raw[off:off + step]).digest()
        cumulative = hashlib.sha256(running + content).digest()
        keys.append(ChunkKey(prefix_key=running, cumulative_key=cumulative))
        running = cumulative
    return keys, running


def compute_prefix_hashes(tokens: list[int], chunk_size: int = DEFAULT_CHUNK_SIZE,
                          initial_salt: bytes = _INITIAL_SALT) -> list[ChunkKey]:
    return _compute(tokens, chunk_size, initial_salt)[0]


def compute_prefix_hashes_and_final(tokens: list[int], chunk_size: int = DEFAULT_CHUNK_SIZE,
                                    initial_salt: bytes = _INITIAL_SALT
                                    ) -> tuple[list[ChunkKey], bytes]:
    """Keys plus the final cumulative hash (the prefix key of the next chunk)."""
    return _compute(tokens, chunk_size, initial_salt)


def longest_prefix_hits(cache_index: dict[bytes, ChunkKey], tokens: list[int],
                        chunk_size: int = DEFAULT_CHUNK_SIZE) -> tuple[list[ChunkKey], int]:
    """Longest run of leading whole chunks of `tokens` present in cache_index.
    Returns (matched keys in order, index of the first unmatched token)."""
    n_full = len(tokens) // chunk_size
    keys, _ = _compute(list(tokens[:n_full * chunk_size]), chunk_size, _INITIAL_SALT)
    matched: list[ChunkKey] = []
    for key in keys:
        if key.full_key not in cache_index:
            break
        matched.append(key)
    return matched, len(matched) * chunk_size
