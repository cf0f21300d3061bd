"""Seeded synthetic inputs from the reference's own generator, regenerable by any host.

The uniform source is the reference sampler's xorshift64* (runtime/sampler.rs:55-75): a state
of 0 becomes 0x9e3779b97f4a7c15; each draw shifts the state by 12 right, 25 left and 27 right
(xor each time) and returns the upper 24 bits of state * 0x2545F4914F6CDD1D divided by 2^24
(an f32 in [0, 1)).

Tensors use many independent streams so that large ones vectorise:

* Stream j of (seed, tag) starts from mix64(mix64(seed ^ (tag << 32)) ^ j), where mix64 is
  the splitmix64 output function (add 0x9E3779B97F4A7C15, then xor-shift-multiply by
  0xBF58476D1CE4E5B9 and 0x94D049BB133111EB with shifts 30, 27, 31).  A zero start becomes
  0x9e3779b97f4a7c15, as in the reference.
* A tensor of n values uses S = min(STREAMS, n) streams.  Value i is draw i // S of stream
  i % S.
* Normals come from Box-Muller on consecutive draws of one stream.  Draws 2p and 2p + 1 give
  u1 and u2; with r = sqrt(-2 ln(1 - u1)), draw 2p is r cos(2 pi u2) and draw 2p + 1 is
  r sin(2 pi u2).  Both are computed in f64 and rounded to f32 (times a scale, also in f64,
  when one is given).
* Integers in [lo, hi] are lo + floor(u * (hi - lo + 1)), with u widened to f64.
* A permutation of range(n) is Fisher-Yates on stream 0 of its tag: for i from n - 1 down to
  1, swap i with floor(u * (i + 1)).
* Tags of named tensors are the CRC-32 (zlib) of the name.

A host with a correctly rounded libm reproduces every value bit for bit.  Elsewhere the f64
transcendentals may differ in their last bit, which changes an f32 value only when it sits
on a rounding boundary.  tests/golden/seeded_inputs.json pins the streams and one value set
per configuration.
"""
from __future__ import annotations

import os
import zlib

import numpy as np

STREAMS = 65536
ZERO_STATE = 0x9E3779B97F4A7C15
MULT = 0x2545F4914F6CDD1D
_M64 = (1 << 64) - 1


def mix64(z: int) -> int:
    """splitmix64's output function of the state before its increment (Python ints)."""
    z = (z + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def _mix64_np(z: np.ndarray) -> np.ndarray:
    z = z + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def tag_of(name: str) -> int:
    return zlib.crc32(name.encode())


def stream_states(seed: int, tag: int, count: int) -> np.ndarray:
    """Start states (uint64) of streams 0..count-1 of (seed, tag)."""
    base = np.uint64(mix64((int(seed) ^ (int(tag) << 32)) & _M64))
    with np.errstate(over="ignore"):
        s = _mix64_np(base ^ np.arange(count, dtype=np.uint64))
    s[s == 0] = np.uint64(ZERO_STATE)
    return s


def next_f32(states: np.ndarray) -> np.ndarray:
    """Advances every stream one draw in place; returns the draws (f32 in [0, 1))."""
    x = states
    x ^= x >> np.uint64(12)
    x ^= x << np.uint64(25)
    x ^= x >> np.uint64(27)
    with np.errstate(over="ignore"):
        upper = (x * np.uint64(MULT)) >> np.uint64(40)
    return upper.astype(np.float32) / np.float32(1 << 24)


def uniforms(seed: int, tag: int, n: int) -> np.ndarray:
    """n uniform f32 draws laid out as the module docstring says."""
    if n == 0:
        return np.zeros(0, np.float32)
    s = min(STREAMS, n)
    st = stream_states(seed, tag, s)
    draws = -(-n // s)
    out = np.empty((draws, s), np.float32)
    for d in range(draws):
        out[d] = next_f32(st)
    return out.reshape(-1)[:n]


def integers(seed: int, tag: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n integers in [lo, hi] (int64)."""
    u = uniforms(seed, tag, n).astype(np.float64)
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)


def normals(seed: int, tag: int, shape, scale: float | None = None, threads: int | None = None) -> np.ndarray:
    """N(0, 1) (times scale) f32 values of the given shape, laid out as the module docstring
    says.  Large tensors split their streams over `threads` threads (default: the host's CPUs,
    at most 16); every stream is independent, so the values do not depend on the split."""
    n = int(np.prod(shape)) if len(shape) else 1
    if n == 0:
        return np.zeros(shape, np.float32)
    s = min(STREAMS, n)
    st = stream_states(seed, tag, s)
    draws = -(-n // s)
    pairs = -(-draws // 2)
    out = np.empty((2 * pairs, s), np.float32)
    two_pi = 2.0 * np.pi

    def fill(c0, c1):
        sub = st[c0:c1].copy()
        for p in range(pairs):
            u1 = next_f32(sub).astype(np.float64)
            u2 = next_f32(sub).astype(np.float64)
            r = np.sqrt(-2.0 * np.log(1.0 - u1))
            z0 = r * np.cos(two_pi * u2)
            z1 = r * np.sin(two_pi * u2)
            if scale is not None:
                z0 *= scale
                z1 *= scale
            out[2 * p, c0:c1] = z0.astype(np.float32)
            out[2 * p + 1, c0:c1] = z1.astype(np.float32)

    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    # narrower streams groups pay more interpreter time per value, so only tensors of 64M
    # values and more are split
    groups = max(1, min(threads, n >> 26, s // 4096))
    if groups == 1:
        fill(0, s)
    else:
        from concurrent.futures import ThreadPoolExecutor

        bounds = [s * g // groups for g in range(groups + 1)]
        with ThreadPoolExecutor(groups) as ex:  # numpy's ufuncs release the GIL
            list(ex.map(lambda g: fill(bounds[g], bounds[g + 1]), range(groups)))
    return out.reshape(-1)[:n].reshape(shape)


def normals_torch(seed: int, tags, shape, scale: float | None = None, device="cuda", out_dtype=None):
    """normals(seed, tag, shape, scale) for every tag of `tags`, stacked ([len(tags), *shape]),
    computed with torch on `device`: the same streams, draws and Box-Muller arithmetic in
    int64 / f64 tensor ops (logical shifts emulated by masking), all tags' streams advanced
    together.  Values equal normals()'s wherever the device's f64 log, sqrt, cos and sin round
    as the host's do (elsewhere an f32 may differ in its last bit).  out_dtype (default f32)
    narrows each drawn row as it is produced, e.g. torch.bfloat16 for bf16 weights."""
    import torch

    out_dtype = torch.float32 if out_dtype is None else out_dtype
    n = int(np.prod(shape)) if len(shape) else 1
    tags = list(tags)
    out = torch.empty((len(tags), n), dtype=out_dtype, device=device)
    if n == 0 or not tags:
        return out.reshape(len(tags), *shape)
    s = min(STREAMS, n)
    st = torch.from_numpy(np.stack([stream_states(seed, t, s) for t in tags]).view(np.int64)).to(device)
    draws = -(-n // s)
    pairs = -(-draws // 2)
    m12 = (1 << 52) - 1  # (x >> 12) as a logical shift
    m27 = (1 << 37) - 1
    m40 = (1 << 24) - 1
    mult = torch.tensor(MULT, dtype=torch.int64, device=device)  # below 2^63; products wrap mod 2^64
    two_pi = 2.0 * np.pi

    def draw():
        nonlocal st
        st = st ^ ((st >> 12) & m12)
        st = st ^ (st << 25)
        st = st ^ ((st >> 27) & m27)
        upper = ((st * mult) >> 40) & m40
        return upper.to(torch.float32) / float(1 << 24)

    view = out.view(len(tags), -1)
    for p in range(pairs):
        u1 = draw().to(torch.float64)
        u2 = draw().to(torch.float64)
        r = torch.sqrt(-2.0 * torch.log(1.0 - u1))
        z = torch.stack((r * torch.cos(two_pi * u2), r * torch.sin(two_pi * u2)), dim=1)  # [tags, 2, s]
        if scale is not None:
            z = z * scale
        z = z.to(torch.float32).reshape(len(tags), 2 * s)
        lo = 2 * p * s
        hi = min(n, lo + 2 * s)
        view[:, lo:hi] = z[:, :hi - lo].to(out_dtype)
    return out.reshape(len(tags), *shape)


def permutation(seed: int, tag: int, n: int) -> np.ndarray:
    """A permutation of range(n) (int32) by Fisher-Yates on stream 0 of (seed, tag)."""
    st = stream_states(seed, tag, 1)
    x = int(st[0])
    perm = list(range(n))
    for i in range(n - 1, 0, -1):
        x ^= x >> 12
        x ^= (x << 25) & _M64
        x ^= x >> 27
        u = ((x * MULT) & _M64) >> 40
        j = int(np.floor(float(np.float32(u) / np.float32(1 << 24)) * (i + 1)))
        perm[i], perm[j] = perm[j], perm[i]
    return np.asarray(perm, np.int32)
