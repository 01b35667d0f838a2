"""rand 0.9 ``StdRng::seed_from_u64`` + ``random::<f32>()``, restated.

The reference's ``get_random_tensors`` (lloom-tensor/tests/quantized_tests.rs
:1267-1287) draws from ``StdRng`` (rand 0.9.x, Cargo.lock: ChaCha12 from
rand_chacha 0.9).  rand's source is not vendored in the reference, so this
follows the published algorithms:
  * rand_core ``SeedableRng::seed_from_u64``: a PCG32 (XSH-RR) stream,
    mul 6364136223846793005, inc 11634580027462260723, fills the 32-byte key
    4 bytes (little endian) at a time;
  * ChaCha with 12 rounds (6 double rounds), 64-bit block counter starting
    at 0 in words 12-13, stream id 0 in words 14-15, output words consumed in
    order (RFC 7539 block function with the original 64/64 split);
  * ``StandardUniform`` for f32: ``(next_u32 >> 8) as f32 * 2^-24``.
Checked against the reference's literal f32 matmul values, see
tests/test_oracle_pins.py.
"""
import numpy as np

M32 = 0xFFFFFFFF


def _pcg32_bytes(state):
    state = (state * 6364136223846793005 + 11634580027462260723) & 0xFFFFFFFFFFFFFFFF
    xorshifted = (((state >> 18) ^ state) >> 27) & M32
    rot = state >> 59
    x = ((xorshifted >> rot) | (xorshifted << ((-rot) & 31))) & M32
    return state, x


def _rotl(v, c):
    return ((v << c) & M32) | (v >> (32 - c))


def _qr(s, a, b, c, d):
    s[a] = (s[a] + s[b]) & M32; s[d] = _rotl(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & M32; s[b] = _rotl(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b]) & M32; s[d] = _rotl(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & M32; s[b] = _rotl(s[b] ^ s[c], 7)


class StdRng:
    def __init__(self, seed_u64):
        state = seed_u64 & 0xFFFFFFFFFFFFFFFF
        key = []
        for _ in range(8):
            state, x = _pcg32_bytes(state)
            key.append(x)
        self.key = key
        self.counter = 0
        self.buf = []

    def _block(self):
        init = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574] + self.key + [
            self.counter & M32, (self.counter >> 32) & M32, 0, 0]
        s = list(init)
        for _ in range(6):
            _qr(s, 0, 4, 8, 12); _qr(s, 1, 5, 9, 13); _qr(s, 2, 6, 10, 14); _qr(s, 3, 7, 11, 15)
            _qr(s, 0, 5, 10, 15); _qr(s, 1, 6, 11, 12); _qr(s, 2, 7, 8, 13); _qr(s, 3, 4, 9, 14)
        self.counter += 1
        return [(s[i] + init[i]) & M32 for i in range(16)]

    def next_u32(self):
        if not self.buf:
            self.buf = self._block()[::-1]
        return self.buf.pop()

    def random_f32(self, count):
        out = np.empty(count, dtype=np.float32)
        scale = np.float32(1.0 / (1 << 24))
        for i in range(count):
            out[i] = np.float32(self.next_u32() >> 8) * scale
        return out
