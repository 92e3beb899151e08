"""std::mt19937_64 (Matsumoto & Nishimura's 64-bit Mersenne Twister with the
constants the C++ standard fixes, [rand.predef]) and the reference sampler's
53-bit uniform (src/generation/sampler.cpp:34-43), for reproducing its draws."""

_N, _M = 312, 156
_A = 0xB5026F5AA96619E9
_UPPER, _LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF
_MASK = (1 << 64) - 1


class MT19937_64:
    def __init__(self, seed=5489):
        self.mt = [0] * _N
        self.mt[0] = seed & _MASK
        for i in range(1, _N):
            self.mt[i] = (6364136223846793005 * (self.mt[i - 1] ^ (self.mt[i - 1] >> 62)) + i) & _MASK
        self.index = _N

    def _twist(self):
        mt = self.mt
        for i in range(_N):
            x = (mt[i] & _UPPER) | (mt[(i + 1) % _N] & _LOWER)
            xa = x >> 1
            if x & 1:
                xa ^= _A
            mt[i] = mt[(i + _M) % _N] ^ xa
        self.index = 0

    def __call__(self):
        if self.index >= _N:
            self._twist()
        y = self.mt[self.index]
        self.index += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & _MASK

    def uniform(self):
        """next_uniform: the top 53 bits of one draw, scaled to [0, 1)."""
        return (self() >> 11) * (1.0 / 9007199254740992.0)
