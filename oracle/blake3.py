"""Test infrastructure only (never imported by the product path): a plain-Python restatement of
BLAKE3 in its default hash mode, the file checksum and tensor key of the reference (blake3==1.0.11,
requirements.txt:7; cli.py:34-39, repo3.py:529, :1029, siblings.py:216-240). The package is absent
here, so this follows the published specification (J. O'Connor, J.-P. Aumasson, S. Neves,
Z. Wilcox-O'Hearn, "BLAKE3: one function, fast everywhere", 2020, sections 2.1-2.6):

  - compression: the 16-word state (chaining value, the first four IV words, counter low/high,
    block length, flags), seven rounds of the ChaCha-style G over columns then diagonals, the
    message words permuted between rounds; output words i ^ i+8 (the chaining value);
  - chunks of 1024 bytes in 64-byte blocks (the last one zero-padded), flags CHUNK_START on the
    first block, CHUNK_END on the last, the chunk index as counter;
  - a binary tree over the chunk chaining values whose left subtree holds the largest power of two
    of chunks strictly below the total (written here as that recursive split: the device and host
    builds pair nodes level by level instead, so the two forms check each other);
  - ROOT on the root's compression (a lone chunk's last block, else the top parent), 32 bytes out.

Pins: the published digests of the empty input and of b"abc" (tests/test_oracle_blake3.py), and the
tree against a second restatement (chaining values pushed on a stack, the specification's
incremental form)."""

IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A, 0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
CHUNK_START, CHUNK_END, PARENT, ROOT = 1, 2, 4, 8
CHUNK, BLOCK = 1024, 64
M32 = 0xFFFFFFFF


def _rotr(x, n):
    return ((x >> n) | (x << (32 - n))) & M32


def _g(s, a, b, c, d, x, y):
    s[a] = (s[a] + s[b] + x) & M32
    s[d] = _rotr(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b] + y) & M32
    s[d] = _rotr(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 7)


def compress(cv, words, counter, blen, flags):
    """the chaining value (8 words) of one compression"""
    s = list(cv) + list(IV[:4]) + [counter & M32, (counter >> 32) & M32, blen, flags]
    m = list(words)
    for r in range(7):
        _g(s, 0, 4, 8, 12, m[0], m[1])
        _g(s, 1, 5, 9, 13, m[2], m[3])
        _g(s, 2, 6, 10, 14, m[4], m[5])
        _g(s, 3, 7, 11, 15, m[6], m[7])
        _g(s, 0, 5, 10, 15, m[8], m[9])
        _g(s, 1, 6, 11, 12, m[10], m[11])
        _g(s, 2, 7, 8, 13, m[12], m[13])
        _g(s, 3, 4, 9, 14, m[14], m[15])
        if r < 6:
            m = [m[PERM[i]] for i in range(16)]
    return [s[i] ^ s[i + 8] for i in range(8)]


def _words(block):
    block = bytes(block) + bytes(BLOCK - len(block))
    return [int.from_bytes(block[4 * i:4 * i + 4], "little") for i in range(16)]


def chunk_cv(data, counter, root=False):
    """chaining value of one chunk (0..1024 bytes); root: its last block carries ROOT"""
    cv = list(IV)
    nb = max(1, -(-len(data) // BLOCK))
    for b in range(nb):
        blk = data[b * BLOCK:(b + 1) * BLOCK]
        flags = (CHUNK_START if b == 0 else 0) | (CHUNK_END if b == nb - 1 else 0)
        if root and b == nb - 1:
            flags |= ROOT
        cv = compress(cv, _words(blk), counter, len(blk), flags)
    return cv


def parent_cv(left, right, root=False):
    return compress(IV, list(left) + list(right), 0, BLOCK, PARENT | (ROOT if root else 0))


def _subtree(data, counter, root):
    """chaining value of the subtree over `data` (a whole number of chunks, but for the last)"""
    n = max(1, -(-len(data) // CHUNK))
    if n == 1:
        return chunk_cv(data, counter, root)
    left = 1 << ((n - 1).bit_length() - 1)            # largest power of two below n
    lcv = _subtree(data[:left * CHUNK], counter, False)
    rcv = _subtree(data[left * CHUNK:], counter + left, False)
    return parent_cv(lcv, rcv, root)


def _out(cv):
    return b"".join(w.to_bytes(4, "little") for w in cv)


def digest(data):
    """the 32-byte BLAKE3 hash of `data` (the recursive form)"""
    return _out(_subtree(bytes(data), 0, True))


def digest_stack(data):
    """the same hash by the specification's incremental form: chunk chaining values pushed on a
    stack, merged while the chunk count is even; the last chunk kept for the root"""
    data = bytes(data)
    n = max(1, -(-len(data) // CHUNK))
    stack = []
    for c in range(n - 1):
        cv = chunk_cv(data[c * CHUNK:(c + 1) * CHUNK], c)
        total = c + 1
        while total & 1 == 0:
            cv = parent_cv(stack.pop(), cv)
            total >>= 1
        stack.append(cv)
    last = data[(n - 1) * CHUNK:]
    if not stack:
        return _out(chunk_cv(last, 0, True))
    cv = chunk_cv(last, n - 1)
    while stack:
        left = stack.pop()
        cv = parent_cv(left, cv, root=not stack)
    return _out(cv)


def hexdigest(data):
    return digest(data).hex()
