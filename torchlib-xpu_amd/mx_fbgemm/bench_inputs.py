"""Seeded synthetic inputs of the benchmark configurations.

Each ``config*`` function returns host (numpy) index data plus the shapes;
large weight tables are generated directly on the device by the caller so
that no multi-GB host copy is needed.  Every function accepts reduced sizes
so the same generator drives the small parity tests.

Configs (numbering of the benchmark plan):
  1  jagged round trip: B=512, lengths U{0..64}, values N(0,1) [sum, 128]
  2  TBE fp32 forward SUM: T=8, E=1e6, D=128, B=4096, L~U{1..40}, Zipf(1.05)
  3  TBE backward + exact rowwise Adagrad on config-2 shapes/indices
  4  nbit MEAN fp16 out: 16 INT8 + 16 INT4 tables, E=1e6, D=128, B=16384, L=20
  5  mixed nbit: 64 tables, D cycling {32,64,128,256}, FP16 / INT4 halves,
     E log-uniform [1e4, 5e6], B=65536, L~Poisson(15) clip [0,100],
     10% empty bags, Zipf(1.1)
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def rng_for(config: int, seed: int = 0, stream: int = 0) -> np.random.Generator:
    ss = np.random.SeedSequence([1000 + config, seed, stream])
    return np.random.default_rng(ss)


def bounded_zipf(rng: np.random.Generator, E: int, a: float, n: int) -> np.ndarray:
    """n draws from P(k) proportional to (k+1)^-a on [0, E), by inverse CDF."""
    w = np.arange(1, E + 1, dtype=np.float64) ** (-a)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = rng.random(n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), E - 1).astype(np.int64)


def offsets_from_lengths(lengths: np.ndarray) -> np.ndarray:
    off = np.zeros(lengths.size + 1, dtype=np.int64)
    np.cumsum(lengths, out=off[1:])
    return off


@dataclass
class JaggedInput:
    values: np.ndarray  # [total_L, D] fp32
    offsets: np.ndarray  # [B+1] int64
    max_L: int


def config1(B: int = 512, D: int = 128, max_L: int = 64, seed: int = 0) -> JaggedInput:
    rng = rng_for(1, seed)
    lengths = rng.integers(0, max_L + 1, size=B)
    off = offsets_from_lengths(lengths)
    values = rng.standard_normal((int(off[-1]), D), dtype=np.float32)
    return JaggedInput(values=values, offsets=off, max_L=max_L)


@dataclass
class TbeInput:
    T: int
    E: list[int]
    D: list[int]
    B: int
    indices: np.ndarray  # int64 [N]
    offsets: np.ndarray  # int64 [T*B+1], t-major

    @property
    def N(self) -> int:
        return int(self.indices.size)

    @property
    def D_offsets(self) -> np.ndarray:
        return offsets_from_lengths(np.asarray(self.D, dtype=np.int64)).astype(np.int32)

    @property
    def total_D(self) -> int:
        return int(sum(self.D))

    @property
    def hash_size_cumsum(self) -> np.ndarray:
        return offsets_from_lengths(np.asarray(self.E, dtype=np.int64))

    @property
    def total_hash_size_bits(self) -> int:
        return max(1, int(int(self.hash_size_cumsum[-1]) - 1).bit_length())


def config2(T: int = 8, E: int = 1_000_000, D: int = 128, B: int = 4096, max_L: int = 40,
            zipf_a: float = 1.05, seed: int = 0) -> TbeInput:
    rng = rng_for(2, seed)
    lengths = rng.integers(1, max_L + 1, size=T * B)
    off = offsets_from_lengths(lengths)
    idx = np.empty(int(off[-1]), dtype=np.int64)
    for t in range(T):
        s, e = int(off[t * B]), int(off[(t + 1) * B])
        perm = rng.permutation(E)
        idx[s:e] = perm[bounded_zipf(rng, E, zipf_a, e - s)]
    return TbeInput(T=T, E=[E] * T, D=[D] * T, B=B, indices=idx, offsets=off)


def config2_batches(k: int, T: int = 8, E: int = 1_000_000, D: int = 128, B: int = 4096,
                    max_L: int = 40, zipf_a: float = 1.05, seed: int = 0) -> list[TbeInput]:
    """k config-2 batches of one model: batch 0 is ``config2(seed=seed)``; the
    others keep its per-table row permutations (the same rows are hot) and
    draw fresh bag lengths and Zipf ranks, as successive training batches do."""
    rng = rng_for(2, seed)
    lengths = rng.integers(1, max_L + 1, size=T * B)
    off = offsets_from_lengths(lengths)
    perms = []
    for t in range(T):  # replays config2's stream to recover its permutations
        perms.append(rng.permutation(E))
        bounded_zipf(rng, E, zipf_a, int(off[(t + 1) * B] - off[t * B]))
    out = [config2(T, E, D, B, max_L, zipf_a, seed)]
    for j in range(1, k):
        r = rng_for(2, seed, stream=j)
        off = offsets_from_lengths(r.integers(1, max_L + 1, size=T * B))
        idx = np.empty(int(off[-1]), dtype=np.int64)
        for t in range(T):
            s, e = int(off[t * B]), int(off[(t + 1) * B])
            idx[s:e] = perms[t][bounded_zipf(r, E, zipf_a, e - s)]
        out.append(TbeInput(T=T, E=[E] * T, D=[D] * T, B=B, indices=idx, offsets=off))
    return out


@dataclass
class NbitInput(TbeInput):
    tys: list[int]  # SparseType ints per table


def config4(T: int = 32, E: int = 1_000_000, D: int = 128, B: int = 16384, L: int = 20,
            seed: int = 0) -> NbitInput:
    rng = rng_for(4, seed)
    off = np.arange(T * B + 1, dtype=np.int64) * L
    idx = rng.integers(0, E, size=T * B * L).astype(np.int64)
    tys = [2] * (T // 2) + [3] * (T - T // 2)  # INT8 then INT4
    return NbitInput(T=T, E=[E] * T, D=[D] * T, B=B, indices=idx, offsets=off, tys=tys)


def config5(T: int = 64, B: int = 65536, e_lo: float = 1e4, e_hi: float = 5e6, lam: float = 15.0,
            max_L: int = 100, empty_frac: float = 0.1, zipf_a: float = 1.1,
            seed: int = 0) -> NbitInput:
    rng = rng_for(5, seed)
    dims = [(32, 64, 128, 256)[t % 4] for t in range(T)]
    tys = [1 if t < T // 2 else 3 for t in range(T)]  # FP16 then INT4
    E = [int(np.floor(np.exp(rng.uniform(np.log(e_lo), np.log(e_hi))))) for _ in range(T)]
    lengths = np.clip(rng.poisson(lam, size=T * B), 0, max_L)
    lengths[rng.random(T * B) < empty_frac] = 0
    off = offsets_from_lengths(lengths)
    idx = np.empty(int(off[-1]), dtype=np.int64)
    for t in range(T):
        s, e = int(off[t * B]), int(off[(t + 1) * B])
        perm = rng.permutation(E[t])
        idx[s:e] = perm[bounded_zipf(rng, E[t], zipf_a, e - s)]
    return NbitInput(T=T, E=E, D=dims, B=B, indices=idx, offsets=off, tys=tys)
