"""Pure-Python BLAKE3, an independent restatement used only to cross-check the C oracle.

TEST INFRASTRUCTURE ONLY (never imported by the product path).

Written from the BLAKE3 specification in its streaming form: chunk states fed byte by byte,
and a chaining-value stack merged by the trailing zero bits of the chunk counter. The C
oracle (oracle/uwc_oracle.c) builds the same tree recursively (left-complete split), and
the GPU kernels reduce it level by level, so the three agree only if all three shapes are
right. The reference's dependency is the `blake3` package (dist/requirements.txt:6),
which is not installed here.
"""
from __future__ import annotations

import struct

IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A, 0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
CHUNK_START, CHUNK_END, PARENT, ROOT, KEYED_HASH = 1, 2, 4, 8, 16
M32 = 0xFFFFFFFF


def _rotr(x: int, n: int) -> int:
    return ((x >> n) | (x << (32 - n))) & M32


def compress(cv, block_words, counter: int, block_len: int, flags: int) -> list[int]:
    s = list(cv) + list(IV[:4]) + [counter & M32, (counter >> 32) & M32, block_len, flags]
    m = list(block_words)

    def g(a, b, c, d, x, y):
        s[a] = (s[a] + s[b] + x) & M32
        s[d] = _rotr(s[d] ^ s[a], 16)
        s[c] = (s[c] + s[d]) & M32
        s[b] = _rotr(s[b] ^ s[c], 12)
        s[a] = (s[a] + s[b] + y) & M32
        s[d] = _rotr(s[d] ^ s[a], 8)
        s[c] = (s[c] + s[d]) & M32
        s[b] = _rotr(s[b] ^ s[c], 7)

    for rnd in range(7):
        g(0, 4, 8, 12, m[0], m[1])
        g(1, 5, 9, 13, m[2], m[3])
        g(2, 6, 10, 14, m[4], m[5])
        g(3, 7, 11, 15, m[6], m[7])
        g(0, 5, 10, 15, m[8], m[9])
        g(1, 6, 11, 12, m[10], m[11])
        g(2, 7, 8, 13, m[12], m[13])
        g(3, 4, 9, 14, m[14], m[15])
        if rnd < 6:
            m = [m[p] for p in PERM]
    return [s[i] ^ s[i + 8] for i in range(8)] + [s[i + 8] ^ cv[i] for i in range(8)]


def _words(block: bytes) -> list[int]:
    return list(struct.unpack("<16I", block.ljust(64, b"\0")))


class _Output:
    def __init__(self, cv, words, counter, blen, flags):
        self.cv, self.words, self.counter, self.blen, self.flags = cv, words, counter, blen, flags

    def chaining_value(self):
        return compress(self.cv, self.words, self.counter, self.blen, self.flags)[:8]

    def root_bytes(self) -> bytes:
        out = compress(self.cv, self.words, 0, self.blen, self.flags | ROOT)[:8]
        return struct.pack("<8I", *out)


class _Chunk:
    def __init__(self, key, counter, flags):
        self.cv, self.counter, self.flags = list(key), counter, flags
        self.buf, self.blocks = b"", 0

    def length(self):
        return 64 * self.blocks + len(self.buf)

    def update(self, data: bytes):
        while data:
            if len(self.buf) == 64:
                fl = self.flags | (CHUNK_START if self.blocks == 0 else 0)
                self.cv = compress(self.cv, _words(self.buf), self.counter, 64, fl)[:8]
                self.blocks += 1
                self.buf = b""
            take = min(64 - len(self.buf), len(data))
            self.buf += data[:take]
            data = data[take:]

    def output(self) -> _Output:
        fl = self.flags | (CHUNK_START if self.blocks == 0 else 0) | CHUNK_END
        return _Output(self.cv, _words(self.buf), self.counter, len(self.buf), fl)


def blake3(data: bytes, key: bytes | None = None) -> bytes:
    """32-byte BLAKE3 digest of data (keyed mode if a 32-byte key is given)."""
    if key is None:
        kw, flags = list(IV), 0
    else:
        assert len(key) == 32
        kw, flags = list(struct.unpack("<8I", key)), KEYED_HASH
    stack: list[list[int]] = []
    chunk = _Chunk(kw, 0, flags)
    pos = 0
    while pos < len(data):
        if chunk.length() == 1024:
            cv = chunk.output().chaining_value()
            total = chunk.counter + 1
            while total & 1 == 0:  # merge completed subtrees
                cv = compress(kw, stack.pop() + cv, 0, 64, PARENT | flags)[:8]
                total >>= 1
            stack.append(cv)
            chunk = _Chunk(kw, chunk.counter + 1, flags)
        take = min(1024 - chunk.length(), len(data) - pos)
        chunk.update(data[pos:pos + take])
        pos += take
    out = chunk.output()
    while stack:
        left = stack.pop()
        out = _Output(kw, left + out.chaining_value(), 0, 64, PARENT | flags)
    return out.root_bytes()
