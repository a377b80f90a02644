"""Oracle for the per-thread random number generator — TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Reference semantics restated (paths relative to /root/reference/src/rdv):
  * shaders/libraries/random_library.h:5-11: one draw advances a uvec4 state
    by three Tausworthe steps (shifts (13, 19, 12), (2, 25, 4), (3, 11, 17),
    masks 0xFFFFFFFE, 0xFFFFFFF8, 0xFFFFFFF0) and one LCG step
    w = 1664525 w + 1013904223 (mod 2^32) — L'Ecuyer's taus88 combined with the
    Numerical Recipes LCG, as in GPU Gems 3 ch. 37 ("hybrid Taus").
  * random_library.h:27-34: random() = float(0x3F800000 | (x^y^z^w) & 0x7FFFFF) - 1,
    a multiple of 2^-23 in [0, 1).
  * random_library.h:49-54 (random_spawn) and :255-267 (the library's per-thread
    init): thread `index` starts from seeds ^ (index ^ 17, index * 123111171,
    index + 11, index ^ (seeds.x + 13 seeds.y)), advanced by one step.
    index = gid.x + 65521 gid.y + 2097143 gid.z; every evaluator here
    dispatches one-dimensionally, so index is the cell / row index.
  * core/_common.py:56-89: one uvec4 of seeds per dispatch.
Everything is uint32 arithmetic modulo 2^32, vectorised over threads.
"""
from __future__ import annotations

import numpy as np

U32 = np.uint32

# (S1, S2, S3, M) of the three Tausworthe components
TAUS = ((13, 19, 12, 0xFFFFFFFE), (2, 25, 4, 0xFFFFFFF8), (3, 11, 17, 0xFFFFFFF0))
LCG_A, LCG_C = 1664525, 1013904223


def taus_step(z, s1: int, s2: int, s3: int, m: int):
    z = np.asarray(z, U32)
    b = ((z << U32(s1)) ^ z) >> U32(s2)
    return ((z & U32(m)) << U32(s3)) ^ b


def lcg_step(z):
    return (np.asarray(z, U32) * U32(LCG_A) + U32(LCG_C)).astype(U32)


def step(state: np.ndarray) -> np.ndarray:
    """One draw's state update; state [..., 4] uint32."""
    s = np.asarray(state, U32)
    out = np.empty_like(s)
    for i, (s1, s2, s3, m) in enumerate(TAUS):
        out[..., i] = taus_step(s[..., i], s1, s2, s3, m)
    out[..., 3] = lcg_step(s[..., 3])
    return out


def spawn(seeds, index) -> np.ndarray:
    """The generator state [n, 4] of threads `index` (int array) of a dispatch."""
    sd = np.asarray(seeds, np.uint64).astype(U32)
    i = np.asarray(index, np.int64).astype(U32)  # the int's bit pattern
    st = np.empty(i.shape + (4,), U32)
    with np.errstate(over="ignore"):
        st[..., 0] = sd[0] ^ (i ^ U32(17))
        st[..., 1] = sd[1] ^ (i * U32(123111171))
        st[..., 2] = sd[2] ^ (i + U32(11))
        st[..., 3] = sd[3] ^ (i ^ (sd[0] + U32(13) * sd[1]))
    return step(st)


def uniform(state: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(random() values float32, new state) of one draw per thread."""
    s = step(state)
    v = s[..., 0] ^ s[..., 1] ^ s[..., 2] ^ s[..., 3]
    f = ((v & U32(0x007FFFFF)) | U32(0x3F800000)).view(np.float32) - np.float32(1.0)
    return f.astype(np.float32), s


def thread_uniforms(seeds, n_threads: int, per_thread: int) -> np.ndarray:
    """[n_threads, per_thread]: each thread's first random() values."""
    st = spawn(seeds, np.arange(n_threads))
    out = np.empty((n_threads, per_thread), np.float32)
    for k in range(per_thread):
        out[:, k], st = uniform(st)
    return out
