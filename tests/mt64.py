"""std::mt19937_64 (Matsumoto and Nishimura, "Mersenne Twister 64-bit",
2004; the C++ standard's [rand.predef] parameters) in Python, for tests that
rebuild seeded models the same way as the C++ fixture generators."""

_MASK = (1 << 64) - 1


class MT19937_64:
    N, M = 312, 156
    A = 0xB5026F5AA96619E9
    UPPER, LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF

    def __init__(self, seed=5489):
        mt = [seed & _MASK]
        for i in range(1, self.N):
            mt.append((6364136223846793005 * (mt[-1] ^ (mt[-1] >> 62)) + i) & _MASK)
        self.mt, self.i = mt, self.N

    def _twist(self):
        mt, N, M = self.mt, self.N, self.M
        for k in range(N):
            x = (mt[k] & self.UPPER) | (mt[(k + 1) % N] & self.LOWER)
            xa = x >> 1
            if x & 1:
                xa ^= self.A
            mt[k] = mt[(k + M) % N] ^ xa
        self.i = 0

    def __call__(self):
        if self.i >= self.N:
            self._twist()
        y = self.mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & _MASK
