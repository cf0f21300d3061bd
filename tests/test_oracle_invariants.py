"""Independent cross-checks of the oracle: closed forms and f64 brute force.

The reference's known-answer vectors (tests/test_oracle_golden.py) pin the oracle's kernels at
tiny shapes (RoPE only at theta 1 with one pair, attention at head_dim 2).  The checks here pin
what those leave open, from the mathematics rather than from a second copy of the loops:

* RoPE (kernel/cpu/attention.rs:165-220, 1242-1292): a unit vector in the low half of pair j
  comes back as (cos a, sin a) with a = pos * theta^(-2j/head_dim) computed in f64, within the
  rounding the f32 recurrence and the f32 angle accumulate; the high half goes to (-sin a, cos a);
  norms are kept; dimensions past rotary_dims pass through unchanged.  Thetas 1e4, 5e5, 1e6 and
  rotary_dims < head_dim, so an exponent over rotary_dims, a sign flip, an interleaved pairing or
  a rotated pass-through band fails.
* Attention (attention.rs:222-686, 729-1149): causal, cached-prefixed, decode and paged decode
  against a brute-force f64 softmax at head_dim 128 and up to 300 keys, 4e-6 normwise (f32
  sequential sums over 128-term dot products and 300 keys; a dropped key, a shifted mask or a
  wrong scale costs > 1e-3); the GQA
  map kv = h / (Hq / Hkv) (a kv = h % Hkv mapping fails); softmax weights are non-negative and
  sum to 1 (values = one-hot rows read the weights back).
* RMSNorm, SwiGLU and the fused greedy head against their f64 definitions at model widths.
"""
import numpy as np
import pytest

import oracle

THETAS = [1e4, 5e5, 1e6]


def f64_inv_freq(theta, head_dim, pairs):
    return np.asarray(theta, np.float64) ** (-2.0 * np.arange(pairs, dtype=np.float64) / head_dim)


@pytest.mark.parametrize("theta", THETAS)
@pytest.mark.parametrize("head_dim,rotary_dims", [(64, 64), (64, 32), (128, 128), (128, 96)])
def test_rope_angles_match_the_closed_form(theta, head_dim, rotary_dims):
    pairs = rotary_dims // 2
    positions = [0, 1, 7, 100, 1023, 2047]
    # probe heads: head 2j carries e_j (low half of pair j), head 2j+1 carries e_(j+pairs)
    # (high half); q rows are [T, heads, D] with one token per probed position
    heads = 2 * pairs
    q = np.zeros((1, heads, head_dim), np.float32)
    for j in range(pairs):
        q[0, 2 * j, j] = 1.0
        q[0, 2 * j + 1, j + pairs] = 1.0
    k = np.zeros((1, 1, head_dim), np.float32)
    inv = f64_inv_freq(theta, head_dim, pairs)
    for pos in positions:
        rq, _ = oracle.rope(q, k, pos, rotary_dims, theta)
        a = pos * inv
        # tolerance: the f32 recurrence inv_(j+1) = inv_j * step drifts by ~(j + 2) ulp, the f32
        # angle adds one more rounding, and sinf / cosf are correctly rounded to ~1 ulp
        tol = pos * inv * (np.arange(pairs) + 4) * 2.0 ** -23 + 4 * 2.0 ** -24
        lo_cos = rq[0, 0::2, :][np.arange(pairs), np.arange(pairs)]
        lo_sin = rq[0, 0::2, :][np.arange(pairs), np.arange(pairs) + pairs]
        hi_sin = rq[0, 1::2, :][np.arange(pairs), np.arange(pairs)]
        hi_cos = rq[0, 1::2, :][np.arange(pairs), np.arange(pairs) + pairs]
        assert np.all(np.abs(lo_cos - np.cos(a)) <= tol), (pos, np.abs(lo_cos - np.cos(a)).max())
        assert np.all(np.abs(lo_sin - np.sin(a)) <= tol), pos
        assert np.all(np.abs(hi_sin + np.sin(a)) <= tol), pos
        assert np.all(np.abs(hi_cos - np.cos(a)) <= tol), pos
        # every other entry of a probe row stays exactly zero (pairing, no leakage)
        mask = np.ones_like(rq, bool)
        for j in range(pairs):
            mask[0, 2 * j, [j, j + pairs]] = False
            mask[0, 2 * j + 1, [j, j + pairs]] = False
        assert np.all(rq[mask] == 0.0)


@pytest.mark.parametrize("theta", THETAS)
def test_rope_exponent_uses_head_dim_not_rotary_dims(theta):
    """With rotary_dims < head_dim the frequency schedule still divides by head_dim: pair 1's
    angle at position 1 is theta^(-2/head_dim), far from theta^(-2/rotary_dims)."""
    head_dim, rotary_dims = 128, 64
    q = np.zeros((1, 1, head_dim), np.float32)
    q[0, 0, 1] = 1.0
    rq, _ = oracle.rope(q, np.zeros((1, 1, head_dim), np.float32), 1, rotary_dims, theta)
    got = np.arctan2(rq[0, 0, 1 + rotary_dims // 2], rq[0, 0, 1])
    assert abs(got - theta ** (-2.0 / head_dim)) < 1e-6
    assert abs(got - theta ** (-2.0 / rotary_dims)) > 1e-2


@pytest.mark.parametrize("theta", THETAS)
def test_rope_preserves_norms_and_passes_through_the_tail(theta):
    rng = np.random.default_rng(5)
    t, hq, hkv, d, rot = 37, 6, 2, 128, 96
    q = rng.standard_normal((t, hq, d), dtype=np.float32)
    k = rng.standard_normal((t, hkv, d), dtype=np.float32)
    rq, rk = oracle.rope(q, k, 900, rot, theta)
    pairs = rot // 2
    for x, rx in ((q, rq), (k, rk)):
        n0 = x[..., :pairs].astype(np.float64) ** 2 + x[..., pairs:rot].astype(np.float64) ** 2
        n1 = rx[..., :pairs].astype(np.float64) ** 2 + rx[..., pairs:rot].astype(np.float64) ** 2
        assert np.allclose(n1, n0, rtol=2e-6, atol=1e-6)
        assert np.array_equal(rx[..., rot:], x[..., rot:])


# ----------------------------------------------------------------------------- attention
def brute_force(q, keys, values, limits):
    """f64 softmax attention: query row t of head h attends keys [0, limits[t]) of kv head
    h // (Hq / Hkv), scale 1/sqrt(D)."""
    t, hq, d = q.shape
    hkv = keys.shape[1]
    g = hq // hkv
    out = np.zeros((t, hq, d), np.float64)
    q64, k64, v64 = (np.asarray(x, np.float64) for x in (q, keys, values))
    for i in range(t):
        n = limits[i]
        for h in range(hq):
            kv = h // g
            s = (k64[:n, kv] @ q64[i, h]) / np.sqrt(d)
            w = np.exp(s - s.max())
            w /= w.sum()
            out[i, h] = w @ v64[:n, kv]
    return out


def rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.abs(ref).max())


ATTN_TOL = 4e-6


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2), (32, 8)])
def test_causal_and_prefixed_attention_against_f64(hq, hkv):
    rng = np.random.default_rng(hq * 10 + hkv)
    d, cache, t = 128, 240, 60
    q = rng.standard_normal((t, hq, d), dtype=np.float32)
    k = rng.standard_normal((cache + t, hkv, d), dtype=np.float32)
    v = rng.standard_normal((cache + t, hkv, d), dtype=np.float32)
    ref = brute_force(q, k, v, [cache + i + 1 for i in range(t)])
    assert rel(oracle.prefixed_causal_attention(q, k, v, cache), ref) <= ATTN_TOL
    # cached-prefixed: cache rows from the cached tensor, the chunk's rows from the suffix
    got = oracle.cached_prefixed_causal_attention(q, k[:cache], v[:cache], cache, k[cache:], v[cache:])
    assert rel(got, ref) <= ATTN_TOL
    # plain causal self-attention over the chunk alone
    ref0 = brute_force(q, k[cache:], v[cache:], [i + 1 for i in range(t)])
    assert rel(oracle.causal_self_attention(q, k[cache:], v[cache:]), ref0) <= ATTN_TOL


def test_gqa_head_mapping_is_blocked():
    """Query head h reads kv head h // (Hq / Hkv): with kv heads holding distinct constant values,
    output head h equals the constant of kv head h // 4 (a h % Hkv mapping would not)."""
    hq, hkv, d, n = 8, 2, 16, 5
    q = np.random.default_rng(0).standard_normal((1, hq, d), dtype=np.float32)
    k = np.random.default_rng(1).standard_normal((n, hkv, d), dtype=np.float32)
    v = np.zeros((n, hkv, d), np.float32)
    v[:, 0, :] = 3.0
    v[:, 1, :] = -5.0
    out = oracle.prefixed_causal_attention(q, k, v, n - 1)
    expect = np.array([3.0 if h // (hq // hkv) == 0 else -5.0 for h in range(hq)], np.float32)
    assert np.allclose(out[0, :, 0], expect, rtol=1e-6)


def test_decode_and_paged_decode_against_f64():
    rng = np.random.default_rng(9)
    hq, hkv, d, cache = 32, 8, 128, 299
    q = rng.standard_normal((1, hq, d), dtype=np.float32)
    ck = rng.standard_normal((cache, hkv, d), dtype=np.float32)
    cv = rng.standard_normal((cache, hkv, d), dtype=np.float32)
    ks = rng.standard_normal((hkv, d), dtype=np.float32)
    vs = rng.standard_normal((hkv, d), dtype=np.float32)
    keys = np.concatenate([ck, ks[None]], 0)
    vals = np.concatenate([cv, vs[None]], 0)
    ref = brute_force(q, keys, vals, [cache + 1])
    assert rel(oracle.decode_causal_attention(q, ck, cv, cache, ks, vs), ref) <= ATTN_TOL
    # the paged gather path over a shuffled page table reaches the same keys
    page = 16
    n = cache + 1
    npages = (n + page - 1) // page
    perm = rng.permutation(64)[:npages].astype(np.int32)
    kp = np.zeros((64, page, hkv, d), np.float32)
    vp = np.zeros_like(kp)
    for i in range(n):
        kp[perm[i // page], i % page] = keys[i]
        vp[perm[i // page], i % page] = vals[i]
    got = oracle.paged_decode_gather_attention(q, kp, vp, perm[None, :], np.array([n], np.int32), page)
    assert rel(got, ref) <= ATTN_TOL


def test_softmax_weights_are_a_distribution():
    """With one-hot value rows (row s = e_s) the output is the weight vector itself: weights are
    non-negative, sum to 1 and equal the f64 softmax."""
    rng = np.random.default_rng(4)
    n, d = 100, 128
    q = rng.standard_normal((1, 4, d), dtype=np.float32) * 2
    k = rng.standard_normal((n, 1, d), dtype=np.float32)
    v = np.zeros((n, 1, d), np.float32)
    v[np.arange(n), 0, np.arange(n)] = 1.0
    out = oracle.prefixed_causal_attention(q, k, v, n - 1)
    w = out[0, :, :n].astype(np.float64)
    assert np.all(w >= 0)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
    assert np.all(out[0, :, n:] == 0)
    ref = brute_force(q, k, v, [n])[0, :, :n]
    assert np.abs(w - ref).max() <= 1e-6


# ----------------------------------------------------------------------------- decoder-block ops
def test_rms_norm_against_f64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((9, 896), dtype=np.float32) * 3
    w = rng.standard_normal(896, dtype=np.float32)
    eps = 1e-6
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * w
    got = oracle.rms_norm(x, w, eps)
    assert rel(got, ref) <= ATTN_TOL


def test_swiglu_against_f64():
    rng = np.random.default_rng(3)
    up = rng.standard_normal(4864, dtype=np.float32) * 4
    gate = rng.standard_normal(4864, dtype=np.float32) * 4
    g64 = gate.astype(np.float64)
    ref = up.astype(np.float64) * (g64 / (1 + np.exp(-g64)))
    got = oracle.mul(up, oracle.silu(gate))
    assert rel(got, ref) <= ATTN_TOL


def test_fused_greedy_head_against_f64():
    """matmul_rhs_transposed_argmax: the first maximal index of h W^T and 1 / sum exp(l - max)."""
    rng = np.random.default_rng(6)
    hidden, vocab = 256, 4096
    h = rng.standard_normal((1, hidden), dtype=np.float32)
    w = rng.standard_normal((vocab, hidden), dtype=np.float32)
    w[1234] = w[99]  # a tie: the first index wins
    h[0] = w[99] * 0.5
    logits = w.astype(np.float64) @ h[0].astype(np.float64)
    idx, prob = oracle.matmul_rhs_transposed_argmax(h, w)
    assert idx == 99
    assert abs(prob - 1.0 / np.exp(logits - logits.max()).sum()) <= 1e-5 * prob
