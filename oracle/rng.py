"""Random streams of the connectivity builders (test infrastructure only).

* ``MT19937``: the generator behind ``numpy.random.RandomState(seed)``, which
  brainstate/nn/_event_fixedprob.py:163-168,186 draws the fixed-num indices and the afferent
  selection from.  Restated from the published algorithm (Matsumoto & Nishimura 1998:
  init_genrand seeding, 624-word twist, tempering), with numpy's legacy bounded integers
  (``randint``: draw = word & mask, mask the smallest 2^j - 1 >= high - 1, redrawn while
  above high - 1; nothing is drawn for a single value) and ``random()`` ((a * 2^26 + b) / 2^53
  from word >> 5 and the next word >> 6).  Pinned against numpy itself in
  tests/test_oracle_rng.py.
* ``philox4x32``: Philox4x32-10 (Salmon, Moraes, Dror & Shaw 2011), the counter-based
  generator of the device's without-replacement sampler, pinned by the Random123 known-answer
  vectors; ``unique_rows`` restates that sampler (K draws per row, Lemire bounded integers,
  redraw the later copy of every repeated value, rows keep draw order).
"""
import numpy as np

_N, _M = 624, 397
_A = np.uint32(0x9908B0DF)
U32 = np.uint32


class MT19937:
    def __init__(self, seed):
        key = np.zeros(_N, np.uint64)
        x = int(seed) & 0xFFFFFFFF
        for i in range(_N):
            key[i] = x
            x = (1812433253 * (x ^ (x >> 30)) + i + 1) & 0xFFFFFFFF
        self.key = key.astype(U32)
        self.pos = _N

    @staticmethod
    def _mix(a, b):
        y = (a & U32(0x80000000)) | (b & U32(0x7FFFFFFF))
        return (y >> U32(1)) ^ np.where((y & U32(1)) != 0, _A, U32(0))

    def _twist(self):
        k = self.key.copy()
        k[:_N - _M] = k[_M:] ^ self._mix(k[:_N - _M], k[1:_N - _M + 1])
        for lo, hi in ((_N - _M, 2 * (_N - _M)), (2 * (_N - _M), _N - 1)):
            k[lo:hi] = k[lo - (_N - _M):hi - (_N - _M)] ^ self._mix(k[lo:hi], k[lo + 1:hi + 1])
        k[_N - 1] = k[_M - 1] ^ self._mix(k[_N - 1:_N], k[0:1])[0]
        self.key = k
        self.pos = 0

    @staticmethod
    def _temper(y):
        y = y.copy()
        y ^= y >> U32(11)
        y ^= (y << U32(7)) & U32(0x9D2C5680)
        y ^= (y << U32(15)) & U32(0xEFC60000)
        y ^= y >> U32(18)
        return y

    def words(self, n):
        """Next n tempered 32-bit outputs."""
        out = np.empty(n, U32)
        got = 0
        while got < n:
            if self.pos == _N:
                self._twist()
            take = min(n - got, _N - self.pos)
            out[got:got + take] = self._temper(self.key[self.pos:self.pos + take])
            self.pos += take
            got += take
        return out

    def randint(self, high, size):
        """numpy's legacy RandomState.randint(0, high, size) (masked rejection)."""
        n = int(np.prod(size))
        rng = high - 1
        if rng == 0:
            return np.zeros(size, np.int64)
        mask = rng
        for s in (1, 2, 4, 8, 16):
            mask |= mask >> s
        parts, need = [], n
        while need > 0:
            if self.pos == _N:
                self._twist()
            v = (self._temper(self.key[self.pos:]) & U32(mask)).astype(np.int64)
            acc = np.flatnonzero(v <= rng)
            if acc.size >= need:
                parts.append(v[acc[:need]])
                self.pos += int(acc[need - 1]) + 1
                need = 0
            else:
                parts.append(v[acc])
                self.pos = _N
                need -= acc.size
        return np.concatenate(parts).reshape(size) if parts else np.zeros(size, np.int64)

    def random(self, n):
        """RandomState.random(n): 53-bit doubles from pairs of words."""
        w = self.words(2 * n).reshape(n, 2)
        a = (w[:, 0] >> U32(5)).astype(np.float64)
        b = (w[:, 1] >> U32(6)).astype(np.float64)
        return (a * 67108864.0 + b) / 9007199254740992.0


# ---- Philox4x32-10 ----

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85


def philox4x32(ctr, key, rounds=10):
    """ctr: uint32 array [..., 4]; key: (k0, k1) uint32 arrays broadcastable to ctr[..., 0]."""
    c = [np.asarray(ctr[..., i], np.uint64) for i in range(4)]
    k0 = np.asarray(key[0], np.uint64) + np.zeros_like(c[0])
    k1 = np.asarray(key[1], np.uint64) + np.zeros_like(c[0])
    m32 = np.uint64(0xFFFFFFFF)
    for _ in range(rounds):
        p0 = np.uint64(_M0) * c[0]
        p1 = np.uint64(_M1) * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ k0) & m32, p1 & m32,
             ((p0 >> np.uint64(32)) ^ c[3] ^ k1) & m32, p0 & m32]
        k0 = (k0 + np.uint64(_W0)) & m32
        k1 = (k1 + np.uint64(_W1)) & m32
    return np.stack([x.astype(U32) for x in c], axis=-1)


def _bounded(seed, row, pos, rnd, n):
    """Lemire's bounded integer for draw (row, pos, round): the first of the four words of
    attempt 0, 1, ... with (word * n) mod 2^32 >= 2^32 mod n gives (word * n) >> 32."""
    thr = (2 ** 32) % n
    k = (seed & 0xFFFFFFFF, seed >> 32)
    for a in range(16):
        r = philox4x32(np.array([row, pos, rnd, a], np.uint64).astype(U32), k)
        for v in r:
            m = int(v) * n
            if (m & 0xFFFFFFFF) >= thr:
                return m >> 32
    return m >> 32


def unique_rows(seed, n_pre, k, n_post):
    """The device's allow_multi_conn=False sampler, row by row (small sizes only)."""
    out = np.zeros((n_pre, k), np.int64)
    for row in range(n_pre):
        val = [_bounded(seed, row, p, 0, n_post) for p in range(k)]
        rnd = [0] * k
        while True:
            order = sorted(range(k), key=lambda p: (val[p], p))
            dup = [order[s] for s in range(1, k) if val[order[s]] == val[order[s - 1]]]
            if not dup:
                break
            for p in dup:
                rnd[p] += 1
                val[p] = _bounded(seed, row, p, rnd[p], n_post)
        out[row] = val
    return out
