"""The seeded input generator (ferrisinfer_amd.seeded) and the BASELINE inputs built on it.

Pins:
* splitmix64 (the stream seeding) against its published output sequence for state 1234567;
* the xorshift64* transition against the oracle's SamplerState, which the reference's own
  sampler tests pin;
* the uniform, normal and integer draws against their distributions (Kolmogorov-Smirnov,
  chi-square) and the permutation against being one;
* the layout rule (value i = draw i // S of stream i % S) against a one-stream recomputation;
* the C1-C4 inputs against the committed fixtures (tests/golden/seeded_inputs.json, written by
  tests/golden/make_seeded_fixtures.py): lengths, ids and ticks exactly, tensors by SHA-256.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from ferrisinfer_amd import seeded

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "seeded_inputs.json")


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_splitmix64_published_sequence():
    # splitmix64 from state 1234567: the reference outputs of the algorithm's published test
    expected = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                16408922859458223821]
    state, got = 1234567, []
    for _ in range(5):
        got.append(seeded.mix64(state))
        state = (state + 0x9E3779B97F4A7C15) % (1 << 64)
    assert got == expected
    # the vectorised form agrees with the scalar one
    z = np.array([1234567, 0, (1 << 64) - 1], np.uint64)
    assert [int(x) for x in seeded._mix64_np(z.copy())] == [seeded.mix64(int(x)) for x in z]


def test_xorshift_transition_matches_the_reference_sampler(orc):
    """One sampled draw of the oracle's SamplerState (pinned by the reference's sampler tests)
    advances the state exactly as seeded.next_f32 does; seed 0 maps to 0x9e3779b97f4a7c15."""
    assert orc.sampler_state_new(0) == seeded.ZERO_STATE
    logits = np.array([0.5, 1.0, -0.25, 2.0], np.float32)
    for s in (1, 42, 0x9E3779B97F4A7C15, (1 << 64) - 1, 123456789123):
        st = np.array([s], np.uint64)
        seeded.next_f32(st)
        _, _, ref_state = orc.sample_last_token(logits, 1.0, 3, 1.0, s)
        assert int(st[0]) == ref_state


def test_draws_follow_their_distributions():
    from scipy import stats

    u = seeded.uniforms(0, 11, 200_000).astype(np.float64)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert stats.kstest(u, "uniform").pvalue > 1e-4
    z = seeded.normals(0, 12, (200_000,)).astype(np.float64)
    assert stats.kstest(z, "norm").pvalue > 1e-4
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    scaled = seeded.normals(0, 12, (200_000,), scale=0.02)
    np.testing.assert_allclose(scaled, (z * 0.02).astype(np.float32), rtol=1e-6, atol=1e-12)
    k = seeded.integers(0, 13, 100_000, 3, 12)
    assert k.min() == 3 and k.max() == 12
    counts = np.bincount(k - 3, minlength=10)
    assert stats.chisquare(counts).pvalue > 1e-4
    p = seeded.permutation(0, 14, 5000)
    assert sorted(p.tolist()) == list(range(5000)) and not np.array_equal(p, np.arange(5000))


def test_layout_rule_streams_and_draws():
    """Value i of an n-value tensor is draw i // S of stream i % S (S = min(STREAMS, n)):
    recomputed stream by stream, and a longer tensor extends a shorter one's streams."""
    n = 10
    u = seeded.uniforms(7, 99, n)  # S = n: one draw per stream
    st = seeded.stream_states(7, 99, n)
    np.testing.assert_array_equal(u, seeded.next_f32(st))
    z = seeded.normals(7, 5, (3 * seeded.STREAMS + 11,))
    st = seeded.stream_states(7, 5, seeded.STREAMS)
    u1 = seeded.next_f32(st).astype(np.float64)
    u2 = seeded.next_f32(st).astype(np.float64)
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    np.testing.assert_array_equal(z[:seeded.STREAMS], (r * np.cos(2 * np.pi * u2)).astype(np.float32))
    np.testing.assert_array_equal(z[seeded.STREAMS:2 * seeded.STREAMS], (r * np.sin(2 * np.pi * u2)).astype(np.float32))


def test_torch_streams_equal_the_numpy_ones():
    """normals_torch (int64 / f64 tensor ops, several tags advanced together) against normals()
    on the host: bit-identical f32 values for short, stream-wide and multi-draw tensors, with and
    without a scale; the bf16 output is the f32 value rounded to nearest even; a split of the
    streams over threads changes nothing."""
    import torch

    for shape, scale in (((7,), 0.02), ((1000,), None), ((300, 500), 0.02), ((2 * seeded.STREAMS + 5,), 0.5)):
        want = np.stack([seeded.normals(3, t, shape, scale=scale) for t in (11, 12, 13)])
        got = seeded.normals_torch(3, [11, 12, 13], shape, scale=scale, device="cpu").numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=str(shape))
    b16 = seeded.normals_torch(3, [11], (4096,), scale=0.02, device="cpu", out_dtype=torch.bfloat16)[0]
    f32 = torch.from_numpy(seeded.normals(3, 11, (4096,), scale=0.02))
    assert torch.equal(b16, f32.to(torch.bfloat16))
    big = (1 << 26) + 3  # long enough to be split over threads
    a = seeded.normals(9, 4, (big,), threads=1)
    b = seeded.normals(9, 4, (big,), threads=4)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_c1_c2_c3_inputs_match_the_fixtures(golden):
    from ferrisinfer_amd import workloads as W

    st = seeded.stream_states(0, 0, 4)
    assert [int(x) for x in st] == golden["streams_seed0_tag0"]["start_states"]
    for d in golden["streams_seed0_tag0"]["draws"]:
        assert seeded.next_f32(st).tolist() == d

    c1 = golden["C1"]
    req = W.c1_requests(0)
    assert [[int(t) for t in p] for p, _ in req] == c1["prompts"]
    assert [m for _, m in req] == c1["max_new_tokens"]
    w = W.random_weights(W.TINY_LLAMA_C1, seed=0)
    assert {k: sha(v) for k, v in w.items()} == c1["weights_sha256"]

    c2g = golden["C2"]
    c2 = W.paged_decode_c2(0)
    assert c2.context_lens.tolist() == c2g["context_lens"]
    assert c2.block_tables[0, :16].tolist() == c2g["first_block_ids"]
    assert sha(c2.block_tables) == c2g["block_tables_sha256"]
    assert sha(c2.q) == c2g["q_sha256"]
    assert sha(c2.k_pool) == c2g["k_pool_sha256"] and sha(c2.v_pool) == c2g["v_pool_sha256"]

    c3g = golden["C3"]
    c3 = W.prefill_c3(0)
    assert c3.prompt_lens.tolist() == c3g["prompt_lens"] and c3.shared_lens.tolist() == c3g["shared_lens"]
    assert sha(c3.block_tables) == c3g["block_tables_sha256"]
    assert (sha(c3.q), sha(c3.k_new), sha(c3.v_new)) == (c3g["q_sha256"], c3g["k_sha256"], c3g["v_sha256"])


def test_c4_inputs_match_the_fixtures(golden):
    """The C4 requests in full; of the 494 M-parameter weights, the embedding and layers 0 and
    23 (the rest follow the same per-name rule)."""
    from ferrisinfer_amd import seeded as S
    from ferrisinfer_amd import workloads as W

    c4g = golden["C4"]
    req = W.c4_requests(0)
    assert [len(r["prompt"]) for r in req] == c4g["prompt_lens"]
    assert [r["max_new_tokens"] for r in req] == c4g["max_new_tokens"]
    assert [r["arrival_tick"] for r in req] == c4g["arrival_ticks"]
    assert sha(np.concatenate([r["prompt"] for r in req])) == c4g["prompt_ids_sha256"]
    cfg = W.QWEN2_05B_C4
    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])
    shapes = {"attention.wq.weight": (h, h), "attention.wk.weight": (h, kvw), "attention.wv.weight": (h, kvw),
              "attention.wq.bias": (h,), "attention.wk.bias": (kvw,), "attention.wv.bias": (kvw,),
              "attention.wo.weight": (h, h), "feed_forward.w1.weight": (h, f),
              "feed_forward.w2.weight": (f, h), "feed_forward.w3.weight": (h, f)}
    names = {"tok_embeddings.weight": (v, h)}
    for layer in (0, cfg["layers"] - 1):
        names.update({f"layers.{layer}.{k}": s for k, s in shapes.items()})
    for name, shape in names.items():
        assert sha(S.normals(0, S.tag_of(name), shape, scale=0.02)) == c4g["weights_sha256"][name], name
