"""BLAKE3: the oracle restatement against published digests, and the library's host hasher
(spa_b3h_*, no GPU needed) against the oracle on every tree shape up to 40 chunks and on pieces of
every alignment."""
import os

import numpy as np
import pytest

from oracle import blake3 as ob

# Published BLAKE3 digests (the first 32 bytes of each output). Inputs of the BLAKE3 project's test
# vectors are the bytes i mod 251 for i < length; b"abc" and b"hello world" are the usual examples.
PUBLISHED = {
    b"": "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262",
    b"abc": "6437b3ac38465133ffb63b75273a8db548c558465d79db03fd359c6cd5bd9d85",
    b"hello world": "d74981efa70a0c880b8d8c1985d075dbcbf679b99a5f9914e5aaf96b831a9e24",
}
VECTORS = {   # length -> digest of bytes(i % 251 for i in range(length))
    1: "2d3adedff11b61f14c886e35afa036736dcd87a74d27b5c1510225d0f592e213",
    1024: "42214739f095a406f3fc83deb889744ac00df831c10daa55189b5d121c855af7",
    1025: "d00278ae47eb27b34faecf67b4fe263f82d5412916c1ffd97c8cb7fb814b8444",
    2048: "e776b6028c7cd22a4d0ba182a8bf62205d2ef576467e838ed6f2529b85fba24a",
    2049: "5f4d72f40d7a5f82b15ca2b2e44b1de3c2ef86c426c95c1af0b6879522563030",
    3072: "b98cb0ff3623be03326b373de6b9095218513e64f1ee2edd2525c7ad1e5cffd2",
    3073: "7124b49501012f81cc7f11ca069ec9226cecb8a2c850cfe644e327d22d3e1cd3",
    4096: "015094013f57a5277b59d8475c0501042c0b642e531b0a1c8f58d2163229e969",
}


def _vec(n):
    return bytes(i % 251 for i in range(n))


def test_oracle_published_digests():
    for data, want in PUBLISHED.items():
        assert ob.hexdigest(data) == want, data
    for n, want in VECTORS.items():
        assert ob.hexdigest(_vec(n)) == want, n


def test_oracle_tree_forms_agree():
    g = np.random.Generator(np.random.PCG64(3))
    for n in (0, 1, 63, 64, 65, 1023, 1024, 1025, 2047, 4097, 5 * 1024 + 7, 9 * 1024, 13 * 1024 + 1):
        d = g.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert ob.digest(d) == ob.digest_stack(d), n


def test_oracle_planted_mistake_fails():
    """a tree whose left subtree is the smaller half (not the largest power of two below the chunk
    count: the odd chunk merged on the left) must miss the published three-chunk digest"""
    def wrong(data, counter, root):
        n = max(1, -(-len(data) // ob.CHUNK))
        if n == 1:
            return ob.chunk_cv(data, counter, root)
        left = n // 2
        return ob.parent_cv(wrong(data[:left * ob.CHUNK], counter, False),
                            wrong(data[left * ob.CHUNK:], counter + left, False), root)
    assert ob._out(wrong(_vec(3072), 0, True)).hex() != VECTORS[3072]
    assert ob._out(wrong(_vec(4096), 0, True)).hex() == VECTORS[4096]      # equal where the split is a power of two


def test_host_hasher_equals_oracle():
    from seedpack_amd import blake3
    g = np.random.Generator(np.random.PCG64(5))
    for nchunks in range(0, 41):
        for extra in (0, 1, 700):
            n = nchunks * 1024 + extra
            d = g.integers(0, 256, n, dtype=np.uint8).tobytes()
            assert blake3.hexdigest(d) == ob.hexdigest(d), n
    for data, want in PUBLISHED.items():
        assert blake3.hexdigest(data) == want


def test_host_hasher_pieces_and_threads():
    from seedpack_amd import blake3
    g = np.random.Generator(np.random.PCG64(6))
    d = g.integers(0, 256, 300 * 1024 + 333, dtype=np.uint8)
    want = ob.hexdigest(d.tobytes())
    for cuts in ([], [1], [1024], [1023, 1025], [5000, 100000, 100001, 250000], list(range(0, len(d), 7777))):
        h = blake3.Hasher(threads=4)
        a = 0
        for c in cuts + [len(d)]:
            h.update(d[a:c])
            a = c
        assert h.hexdigest() == want, cuts
        assert h.hexdigest() == want                 # final leaves the state as it was
    for t in (1, 3, 16):
        assert blake3.hexdigest(d, threads=t) == want
