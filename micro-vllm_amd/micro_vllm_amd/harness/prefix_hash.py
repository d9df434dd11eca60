"""Full-block prefix-cache identities and their per-step host cost.

Restates the reference's block hash (core/prefix_cache.py:12-40): a 32-byte
blake2b digest, personalised with ``micro-vllm-kv``, over

    len(namespace) (8 bytes, big-endian) | namespace (UTF-8) |
    cache_group_id (8) | block_size (8) |
    0x00                      for the first block, or
    0x01 | parent digest      for every later block |
    each token id (8 bytes, big-endian)

so every block's digest chains the whole prefix before it.

The reference recomputes a request's chain from its first block on every
call (core/cache_group_manager.py:193-212), and it caches each request's
computed blocks after every step (core/kv_cache_manager.py:230-248; the full
blocks of ``num_computed_tokens``, cache_group_manager.py:98-132). At the
Llama-3-8B e2e configuration (contexts of 8k-33k tokens, block 16) that is
up to ~2,000 digests per request per step. ``BlockHashChain`` keeps a
request's digests and hashes only blocks that became full since the last
call; its digests are identical, and the semantics of caching do not change.
``measure_step_cost`` times both on such a batch.
"""

from __future__ import annotations

import time
from collections.abc import Sequence
from hashlib import blake2b

import numpy as np

BLOCK_HASH_BYTES = 32
_HASH_DOMAIN = b"micro-vllm-kv"


def hash_block(
    parent_block_hash: bytes | None,
    token_ids: Sequence[int],
    *,
    block_size: int,
    cache_namespace: str,
    cache_group_id: int = 0,
) -> bytes:
    """Digest of one complete token block chained to its parent's digest."""

    namespace = cache_namespace.encode("utf-8")
    digest = blake2b(digest_size=BLOCK_HASH_BYTES, person=_HASH_DOMAIN)
    digest.update(len(namespace).to_bytes(8, "big"))
    digest.update(namespace)
    digest.update(cache_group_id.to_bytes(8, "big"))
    digest.update(block_size.to_bytes(8, "big"))
    if parent_block_hash is None:
        digest.update(b"\x00")
    else:
        digest.update(b"\x01")
        digest.update(parent_block_hash)
    # One token at a time, as the reference does, so that the measured cost
    # per digest is the reference's (int.to_bytes refuses negative ids).
    for token_id in token_ids:
        digest.update(int(token_id).to_bytes(8, "big"))
    return digest.digest()


def block_hashes(
    token_ids: Sequence[int], num_blocks: int, *, block_size: int, cache_namespace: str, cache_group_id: int = 0
) -> tuple[bytes, ...]:
    """The first ``num_blocks`` digests of a token sequence, from scratch, as
    the reference computes them on every call."""

    parent: bytes | None = None
    out = []
    for b in range(num_blocks):
        parent = hash_block(
            parent,
            token_ids[b * block_size : (b + 1) * block_size],
            block_size=block_size,
            cache_namespace=cache_namespace,
            cache_group_id=cache_group_id,
        )
        out.append(parent)
    return tuple(out)


class BlockHashChain:
    """One request's block digests, extended as its blocks fill up.

    With ``vectorized=True`` a block's token ids are encoded in one numpy
    call and fed to a copy of a digest primed with the fixed header: the same
    bytes in the same order, so the digests are identical to ``hash_block``'s
    (blake2b of a concatenation does not depend on how it is split into
    updates)."""

    __slots__ = ("block_size", "cache_namespace", "cache_group_id", "hashes", "_header")

    def __init__(
        self, *, block_size: int, cache_namespace: str, cache_group_id: int = 0, vectorized: bool = False
    ) -> None:
        self.block_size = block_size
        self.cache_namespace = cache_namespace
        self.cache_group_id = cache_group_id
        self.hashes: list[bytes] = []
        self._header = None
        if vectorized:
            namespace = cache_namespace.encode("utf-8")
            header = blake2b(digest_size=BLOCK_HASH_BYTES, person=_HASH_DOMAIN)
            header.update(len(namespace).to_bytes(8, "big"))
            header.update(namespace)
            header.update(cache_group_id.to_bytes(8, "big"))
            header.update(block_size.to_bytes(8, "big"))
            self._header = header

    def extend(self, token_ids: Sequence[int], num_blocks: int) -> tuple[bytes, ...]:
        """The first ``num_blocks`` digests; only blocks not hashed before are
        hashed now. ``token_ids`` must extend the tokens of earlier calls (a
        request's tokens only grow), and every token of the hashed blocks must
        be a real (non-negative) id."""

        bs = self.block_size
        parent = self.hashes[-1] if self.hashes else None
        first = len(self.hashes)
        if self._header is not None and num_blocks > first:
            block_bytes = np.asarray(token_ids[first * bs : num_blocks * bs], dtype=">i8")
            if block_bytes.size and block_bytes.min() < 0:
                raise ValueError("cannot hash a block that holds a negative token id")
            raw = block_bytes.tobytes()
            width = 8 * bs
            for i, b in enumerate(range(first, num_blocks)):
                digest = self._header.copy()
                if parent is None:
                    digest.update(b"\x00")
                else:
                    digest.update(b"\x01")
                    digest.update(parent)
                digest.update(raw[i * width : (i + 1) * width])
                parent = digest.digest()
                self.hashes.append(parent)
            return tuple(self.hashes[:num_blocks])
        for b in range(first, num_blocks):
            parent = hash_block(
                parent,
                token_ids[b * bs : (b + 1) * bs],
                block_size=bs,
                cache_namespace=self.cache_namespace,
                cache_group_id=self.cache_group_id,
            )
            self.hashes.append(parent)
        return tuple(self.hashes[:num_blocks])


def measure_step_cost(
    context_lengths: Sequence[int], *, block_size: int = 16, steps: int = 3, seed: int = 0
) -> dict:
    """Host time to cache the full blocks of every request after one decode
    step: the reference's from-scratch chains against ``BlockHashChain``.

    Each request holds ``context_lengths[r]`` computed tokens; a decode step
    adds one token to each. The chains are primed with the contexts first, so
    the incremental figure is the steady-state cost of a step."""

    rng = np.random.default_rng(seed)
    tokens = [rng.integers(0, 128_256, size=int(n) + steps).tolist() for n in context_lengths]
    namespace = "llama3-8b"
    chains = [BlockHashChain(block_size=block_size, cache_namespace=namespace) for _ in tokens]
    for chain, toks, n in zip(chains, tokens, context_lengths):
        chain.extend(toks, int(n) // block_size)
    scratch, incremental = [], []
    for step in range(1, steps + 1):
        start = time.perf_counter()
        for toks, n in zip(tokens, context_lengths):
            block_hashes(toks, (int(n) + step) // block_size, block_size=block_size, cache_namespace=namespace)
        scratch.append(time.perf_counter() - start)
        start = time.perf_counter()
        for chain, toks, n in zip(chains, tokens, context_lengths):
            chain.extend(toks, (int(n) + step) // block_size)
        incremental.append(time.perf_counter() - start)
    blocks = sum(int(n) // block_size for n in context_lengths)
    return {
        "requests": len(context_lengths),
        "full_blocks": blocks,
        "from_scratch_ms_per_step": round(float(np.median(scratch)) * 1e3, 3),
        "incremental_ms_per_step": round(float(np.median(incremental)) * 1e3, 4),
    }
