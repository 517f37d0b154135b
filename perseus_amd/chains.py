"""Parameter chains of the key-switch / NTT workloads.

A chain is nq Q primes then kp special primes, all = 1 mod 2N and below 2^31 (the u32 word's limit,
crates/pc-core/src/modmul.rs:376-383), with dnum hybrid digits of ceil(nq / dnum) limbs
(crates/pc-core/src/params.rs:500-510). The workloads fix their primes directly, as the reference's `Chain` fields
allow (crates/pc-core/src/params.rs:215-241): descending NTT-friendly primes of a given width, found the way
OpenFHE's LastPrime / PreviousPrime find them (crates/pc-core/src/params/nbtheory.rs:66-107).
"""
from dataclasses import dataclass, field
from typing import List

_WITNESSES = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)


def is_prime(n: int) -> bool:
    """Deterministic Miller-Rabin for every 64-bit n (bases 2..37)."""
    if n < 2:
        return False
    for p in _WITNESSES:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for a in _WITNESSES:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def last_prime(bits: int, m: int) -> int:
    """The largest prime q = 1 mod m below 2^bits."""
    q = 1 << bits
    c = q + 1 - q % m
    if q % m < 2:
        c -= m
    while not is_prime(c):
        c -= m
    return c


def descending_primes(bits: int, m: int, n: int) -> List[int]:
    out, q = [], last_prime(bits, m)
    while len(out) < n:
        if q.bit_length() != bits:
            raise ValueError(f"fewer than {n} {bits}-bit primes = 1 mod {m}")
        out.append(q)
        q -= m
        while not is_prime(q):
            q -= m
    return out


@dataclass
class Chain:
    name: str
    logn: int
    q: List[int]
    p: List[int] = field(default_factory=list)
    dnum: int = 1

    @property
    def n(self) -> int:
        return 1 << self.logn

    @property
    def primes(self) -> List[int]:
        return self.q + self.p

    @property
    def rows(self) -> int:
        return len(self.q) + len(self.p)

    @property
    def alpha(self) -> int:
        return -(-len(self.q) // self.dnum)


def make(name, logn, nq, kp, dnum, bits):
    ps = descending_primes(bits, 2 << logn, nq + kp)
    return Chain(name, logn, ps[:nq], ps[nq:], dnum)


def preset(name: str) -> Chain:
    """The workloads' chains.

    c1: one rotation at N = 2^14, 12 Q primes below 2^30 (lazy butterflies legal), dnum 3, 4 special primes;
    c2: the batched NTT round trip, N = 2^16, 40 primes below 2^31;
    c3: the hoisted rotation batch, N = 2^16, 30 Q primes below 2^31, dnum 3, 6 special primes;
    c4: attention scoring, N = 2^16, 6 Q + 2 special 30-bit primes, dnum 3 (a ciphertext at scale 2^40 takes one
        plaintext product and a two-prime rescale, then its rotations at 4 limbs);
    c5: the full-slot bootstrap, N = 2^16, 47 Q primes below 2^30 (q0, 17 two-prime levels the bootstrap consumes,
        12 limbs left), dnum 3, 16 special primes (as many as a digit's limbs, so key switching adds little noise);
    small: a quick test chain, N = 2^12, 6 Q + 2 special 30-bit primes, dnum 3;
    small28: the same at 28-bit primes (a bootstrapping stage's word size);
    rej: N = 2^12, 6 Q + 3 special primes just above 2^32 / 3, where a third of the KSKA words are rejected.
    """
    if name == "c1":
        return make("c1", 14, 12, 4, 3, 30)
    if name == "c2":
        return make("c2", 16, 40, 0, 1, 31)
    if name == "c3":
        return make("c3", 16, 30, 6, 3, 31)
    if name == "c4":
        return make("c4", 16, 6, 2, 3, 30)
    if name == "c5":
        return make("c5", 16, 47, 16, 3, 30)
    if name == "small":
        return make("small", 12, 6, 2, 3, 30)
    if name == "small28":
        return make("small28", 12, 6, 2, 3, 28)
    if name == "small31":
        return make("small31", 12, 6, 3, 3, 31)
    if name == "rej":
        return Chain("rej", 12, *_split(ascending_primes(2**32 // 3 + 1, 2 << 12, 9), 6), 3)
    raise KeyError(name)


def ascending_primes(lo: int, m: int, n: int) -> List[int]:
    """n primes q = 1 mod m from lo upwards (a test chain: just above 2^32 / 3 a third of the KSKA words are rejected)."""
    out, q = [], (lo + m - 2) // m * m + 1
    while len(out) < n:
        if is_prime(q):
            out.append(q)
        q += m
    return out


def _split(ps, nq):
    return ps[:nq], ps[nq:]
