"""Pins the random-number oracle (oracle/random.py) by what the mathematics and
published tables fix, not by restating its formulas.  CPU only.

  * The LCG component is the Numerical Recipes generator
    (a = 1664525, c = 1013904223): from 0 it must give the sequence printed in
    Numerical Recipes in C (2nd ed., section 7.1).
  * Each Tausworthe component is one of L'Ecuyer's taus88 components, a
    maximal-period linear recurrence over GF(2) on its top k = 31, 29, 28 bits:
    the step's 32x32 bit matrix A satisfies A^(2^k) = A, and no proper divisor
    (2^k - 1) / p of the period does.  A swapped shift, a wrong mask or a wrong
    shift amount breaks this.
  * random() maps 23 random bits to [0, 1) exactly: every value is a multiple
    of 2^-23 in [0, 1), and a long sequence is uniform.
"""
import numpy as np

from oracle import random as R

NR_LCG_FROM_ZERO = [0x3C6EF35F, 0x47502932, 0xD1CCF6E9, 0xAAF95334, 0x6252E503, 0x9F2EC686, 0x57FE6C2D,
                    0xA3D95FA8, 0x81FDBEE7, 0x94F0AF1A, 0xCBF633B1]


def test_lcg_matches_numerical_recipes():
    z = np.zeros(1, np.uint32)
    got = []
    for _ in NR_LCG_FROM_ZERO:
        z = R.lcg_step(z)
        got.append(int(z[0]))
    assert got == NR_LCG_FROM_ZERO


def _bit_matrix(comp: int) -> np.ndarray:
    s1, s2, s3, m = R.TAUS[comp]
    A = np.zeros((32, 32), np.int64)
    for j in range(32):
        v = int(R.taus_step(np.array([1 << j], np.uint32), s1, s2, s3, m)[0])
        A[:, j] = [(v >> i) & 1 for i in range(32)]
    return A


def _gf2_pow(A: np.ndarray, e: int) -> np.ndarray:
    out = np.eye(A.shape[0], dtype=np.int64)
    b = A.copy()
    while e:
        if e & 1:
            out = (out @ b) % 2
        b = (b @ b) % 2
        e >>= 1
    return out


def test_tausworthe_components_have_maximal_period():
    # (component, k, prime factors of 2^k - 1)
    cases = [(0, 31, [2 ** 31 - 1]), (1, 29, [233, 1103, 2089]), (2, 28, [3, 5, 29, 43, 113, 127])]
    for comp, k, primes in cases:
        N = 2 ** k - 1
        assert int(np.prod(primes)) == N
        A = _bit_matrix(comp)
        assert (_gf2_pow(A, N + 1) == A).all(), f"component {comp}: period does not divide 2^{k} - 1"
        for p in primes:
            assert not (_gf2_pow(A, N // p + 1) == A).all(), f"component {comp}: period divides (2^{k} - 1) / {p}"


def test_uniform_values_are_23_bit_fractions():
    u = R.thread_uniforms([1234, 5678, 91011, 121314], 4096, 8)
    assert u.dtype == np.float32
    assert (u >= 0).all() and (u < 1).all()
    scaled = u.astype(np.float64) * 2 ** 23
    assert (scaled == np.floor(scaled)).all()
    # uniformity: 64 bins over 32768 draws, chi-square far below its 1e-6 tail (~130 for 63 dof)
    hist = np.bincount((u.reshape(-1) * 64).astype(np.int64), minlength=64)
    e = u.size / 64
    assert ((hist - e) ** 2 / e).sum() < 130
    # successive draws of one thread are uncorrelated.  (Neighbouring threads'
    # early draws are not: the reference's spawn xors the index into the seeds
    # and takes one step, which leaves |corr| up to ~0.3 between threads i and
    # i + 1 in the first few draws.  That is the reference's generator, kept.)
    # (pooled over 7 x 4096 pairs: the standard error is ~0.006)
    assert abs(np.corrcoef(u[:, :-1].reshape(-1), u[:, 1:].reshape(-1))[0, 1]) < 0.03


def test_spawn_separates_threads_and_dispatches():
    st = R.spawn([128, 129, 130, 131], np.arange(100000))
    keys = st.view(np.uint64).reshape(-1, 2)
    assert np.unique(keys, axis=0).shape[0] == 100000
    a = R.thread_uniforms([128, 129, 130, 131], 256, 2)
    b = R.thread_uniforms([128, 129, 130, 132], 256, 2)
    assert (a != b).mean() > 0.99
    # the first draw after spawn is one step past the spawned state
    s0 = R.spawn([5, 6, 7, 8], np.array([3]))
    f, s1 = R.uniform(s0)
    assert (s1 == R.step(s0)).all()
