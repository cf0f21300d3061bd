"""Pins the CPU oracle to the reference's own known-answer tests.

Every expected vector below is the literal the reference asserts in its #[cfg(test)]
modules (file:line cited per test), with the reference's tolerance.
"""
import numpy as np
import pytest


def approx(a, b, tol):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    assert a.shape == b.shape
    assert np.all(np.abs(a - b) <= tol), (a, b)


# ---- crates/ferrisinfer-kernel/src/cpu/attention.rs tests ----
def test_embedding_gather_selects_rows(orc):
    # attention.rs:1310-1322
    e = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    assert orc.embedding_gather(e, [2, 0]).reshape(-1).tolist() == [5, 6, 1, 2]


def test_embedding_gather_rejects_out_of_vocab(orc):
    # attention.rs:35-40
    with pytest.raises(orc.OracleError) as e:
        orc.embedding_gather(np.zeros((3, 2), np.float32), [3])
    assert e.value.kind == "InvalidShape"


def test_rope_rotates_query_and_key_pairs(orc):
    # attention.rs:1324-1345
    q = np.array([1, 0, 1, 0], np.float32).reshape(2, 1, 2)
    qr, kr = orc.rope(q, q.copy(), 0, 2, 1.0)
    approx(qr, [1.0, 0.0, 0.5403023, 0.84147096], 1e-6)
    approx(kr, [1.0, 0.0, 0.5403023, 0.84147096], 1e-6)


def test_causal_self_attention_respects_mask(orc):
    # attention.rs:1347-1365
    q = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    approx(orc.causal_self_attention(q, q, q), [1.0, 0.0, 0.33023846, 0.66976154], 1e-6)


def test_prefixed_causal_attention_uses_cached_prefix(orc):
    # attention.rs:1367-1382
    q = np.array([0, 1], np.float32).reshape(1, 1, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    approx(orc.prefixed_causal_attention(q, k, k, 1), [0.33023846, 0.66976154], 1e-6)


def test_cached_prefixed_matches_prefixed(orc):
    # attention.rs:1383-1431
    q = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    ck = np.array([1, 1, 0, 0, 0, 0, 0, 0], np.float32).reshape(4, 1, 2)
    ks = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    full = np.array([1, 1, 1, 0, 0, 1], np.float32).reshape(3, 1, 2)
    a = orc.cached_prefixed_causal_attention(q, ck, ck, 1, ks, ks)
    b = orc.prefixed_causal_attention(q, full, full, 1)
    approx(a, b, 1e-6)


def test_decode_matches_prefixed(orc):
    # attention.rs:1433-1478
    q = np.array([1, 0, 0, 1], np.float32).reshape(1, 2, 2)
    ck = np.array([1, 0, 0, 0, 0, 0, 0, 0], np.float32).reshape(4, 1, 2)
    slot = np.array([0, 1], np.float32).reshape(1, 2)
    full = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    a = orc.decode_causal_attention(q, ck, ck, 1, slot, slot)
    b = orc.prefixed_causal_attention(q, full, full, 1)
    approx(a, b, 1e-6)


def test_causal_self_attention_gqa(orc):
    # attention.rs:1480-1504
    q = np.array([1, 0, 1, 0, 0, 1, 0, 1], np.float32).reshape(2, 2, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(2, 1, 2)
    approx(orc.causal_self_attention(q, k, k),
           [1.0, 0.0, 1.0, 0.0, 0.33023846, 0.66976154, 0.33023846, 0.66976154], 1e-6)


# ---- crates/ferrisinfer-kernel/src/cpu/matmul.rs tests ----
def test_matmul_multiplies(orc):
    # matmul.rs:695-712
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert orc.matmul(a, b).reshape(-1).tolist() == [58.0, 64.0, 139.0, 154.0]


def test_matmul_rhs_transposed(orc):
    # matmul.rs:726-743
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8, 9], [10, 11, 12]], np.float32)
    assert orc.matmul_rhs_transposed(a, b).reshape(-1).tolist() == [50.0, 68.0, 122.0, 167.0]


def test_matmul_rhs_transposed_argmax(orc):
    # matmul.rs:745-758
    idx, prob = orc.matmul_rhs_transposed_argmax([[1, 2]], [[1, 0], [0, 1], [1, 1]])
    assert idx == 2
    assert abs(prob - 0.66524094) <= 1e-6


# ---- crates/ferrisinfer-kernel/src/cpu/reduction.rs tests ----
def test_rms_norm(orc):
    # reduction.rs:196-213
    out = orc.rms_norm(np.array([[3, 4], [0, 5]], np.float32), [1.0, 1.5], 1e-5)
    approx(out, [0.84852797, 1.697056, 0.0, 2.1213198], 1e-5)


# ---- crates/ferrisinfer-kernel/src/cpu/elementwise.rs tests ----
def test_add_mul_silu(orc):
    # elementwise.rs:296-357
    assert orc.add([1.0, 2.0, 3.0], [0.5, -1.0, 2.0]).tolist() == [1.5, 1.0, 5.0]
    assert orc.mul([2.0, -3.0, 4.0], [0.5, 2.0, -1.5]).tolist() == [1.0, -6.0, -6.0]
    approx(orc.silu([-1.0, 0.0, 1.0]), [-0.26894143, 0.0, 0.7310586], 1e-6)


# ---- crates/ferrisinfer-runtime/src/reference.rs tests ----
def test_linear_with_bias(orc):
    # reference.rs:1250-1265
    out = orc.linear_with_bias([[1, 2]], [[1, 0], [0, 1]], [0.5, -1.0])
    approx(out, [1.5, 1.0], 1e-6)


def tiny_reference_model(orc):
    """reference.rs:1715-1837 tiny_reference_model: hidden 2, identity attention, zero MLP."""
    m = orc.Model(hidden=2, intermediate=2, layers=1, heads=1, kv_heads=1, vocab=2, max_pos=16,
                  eps=1e-5, theta=10000.0, rotary_dims=0, tie=False)
    eye = np.eye(2, dtype=np.float32)
    z = np.zeros((2, 2), np.float32)
    m.set_weights({
        "tok_embeddings.weight": eye, "layers.0.attention_norm.weight": [1, 1],
        "layers.0.attention.wq.weight": eye, "layers.0.attention.wk.weight": eye,
        "layers.0.attention.wv.weight": eye, "layers.0.attention.wo.weight": eye,
        "layers.0.ffn_norm.weight": [1, 1], "layers.0.feed_forward.w1.weight": z,
        "layers.0.feed_forward.w2.weight": z, "layers.0.feed_forward.w3.weight": z,
        "norm.weight": [1, 1], "output.weight": eye,
    })
    return m


def test_block_forward_single_reference_block(orc):
    # reference.rs:1267-1325: a 1-layer model without final norm effects is not available
    # through the model API, so the block is composed from the oracle's block ops in the
    # reference's order (rmsnorm -> qkv -> attention -> wo -> +x -> rmsnorm -> mlp -> +h1).
    x = np.array([[1, 0], [0, 1]], np.float32)
    normed = orc.rms_norm(x, [1, 1], 1e-5)
    q = normed.reshape(2, 1, 2)
    attn = orc.causal_self_attention(q, q, q).reshape(2, 2)
    h1 = orc.add(attn, x)
    out = orc.add(np.zeros_like(h1), h1)
    approx(out, [2.4141994, 0.0, 0.27658173, 2.1376176], 1e-5)


def test_model_forward_complete_reference_path(orc):
    # reference.rs:1401-1411
    m = tiny_reference_model(orc)
    approx(m.forward_logits([0, 1]), [1.4142112, 0.0, 0.18146895, 1.4025193], 1e-5)


def test_gqa_block_via_model(orc):
    # reference.rs:1327-1399 (GQA block) checked through a 1-layer GQA model whose final
    # norm and output are identity-like: logits = rmsnorm(block_out) · I.
    m = orc.Model(hidden=4, intermediate=2, layers=1, heads=2, kv_heads=1, vocab=4, max_pos=16,
                  eps=0.0, theta=10000.0, rotary_dims=0, tie=False)
    eye4 = np.eye(4, dtype=np.float32)
    kvw = np.array([[1, 0], [0, 1], [0, 0], [0, 0]], np.float32)
    emb = np.zeros((4, 4), np.float32)
    emb[0] = [1.4142135, 0.0, 0.0, 1.4142135]
    m.set_weights({
        "tok_embeddings.weight": emb, "layers.0.attention_norm.weight": np.ones(4),
        "layers.0.attention.wq.weight": eye4, "layers.0.attention.wk.weight": kvw,
        "layers.0.attention.wv.weight": kvw, "layers.0.attention.wo.weight": eye4,
        "layers.0.ffn_norm.weight": np.ones(4), "layers.0.feed_forward.w1.weight": np.zeros((4, 2)),
        "layers.0.feed_forward.w2.weight": np.zeros((2, 4)),
        "layers.0.feed_forward.w3.weight": np.zeros((4, 2)),
        "norm.weight": np.ones(4), "output.weight": eye4,
    })
    logits = m.forward_logits([0])
    block_out = np.array([2.828427, 0.0, 1.4142135, 1.4142135], np.float32)
    expected = orc.rms_norm(block_out[None, :], np.ones(4), 0.0)
    approx(logits, expected, 1e-5)


def test_decode_with_kv_matches_full_forward(orc):
    # reference.rs:1413-1465 (contiguous) and 1467-1505 (paged)
    m = tiny_reference_model(orc)
    full = m.forward_logits([0, 1])[-1]
    for page in (0, 2):
        s = orc.Session(m, max_seq=8, max_gen=8, page_size=page)
        s.prefill([0])
        s.prefill([1])
        hidden = s.last_hidden()
        logits = orc.matmul_rhs_transposed(hidden[None, :], np.eye(2, dtype=np.float32))
        approx(logits, full, 1e-5)
        assert s.position == 2


def test_prefill_with_existing_kv_matches_full(orc):
    # reference.rs:1577-1644
    m = tiny_reference_model(orc)
    full = m.forward_logits([0, 1, 0])[-1]
    for page in (0, 2):
        s = orc.Session(m, max_seq=8, max_gen=8, page_size=page)
        s.prefill([0])
        s.prefill([1, 0])
        logits = orc.matmul_rhs_transposed(s.last_hidden()[None, :], np.eye(2, dtype=np.float32))
        approx(logits, full, 1e-5)
        assert s.position == 3


def test_imported_paged_prefix_matches_full(orc):
    # reference.rs:1646-1675
    m = tiny_reference_model(orc)
    src = orc.Session(m, max_seq=8, max_gen=8, page_size=2)
    src.prefill([0, 1])
    dst = orc.Session(m, max_seq=8, max_gen=8, page_size=2)
    dst.copy_prefix_from(src, 2)
    dst.prefill([0])
    logits = orc.matmul_rhs_transposed(dst.last_hidden()[None, :], np.eye(2, dtype=np.float32))
    approx(logits, m.forward_logits([0, 1, 0])[-1], 1e-5)


def test_fused_argmax_matches_logits_argmax(orc):
    # reference.rs:1507-1547, 1677-1713
    m = tiny_reference_model(orc)
    s = orc.Session(m, max_seq=8, max_gen=8, page_size=0)
    s.prefill([0, 1])
    tok, prob = s.last_sample()
    logits = m.forward_logits([0, 1])
    etok, eprob = orc.argmax_last_token(logits)
    assert tok == etok
    assert abs(prob - eprob) <= 1e-6


# ---- crates/ferrisinfer-runtime/src/paged_kv.rs tests ----
KEYS5 = np.array([1, 2, 5, 6, 9, 10, 13, 14, 17, 18], np.float32).reshape(5, 1, 2)
VALS5 = np.array([3, 4, 7, 8, 11, 12, 15, 16, 19, 20], np.float32).reshape(5, 1, 2)


def test_paged_storage_round_trip_across_pages(orc):
    # paged_kv.rs:922-967
    s = orc.PagedKvStorage(1, 1, 2, 8, 2)
    s.write_sequence(0, 0, KEYS5, VALS5)
    k, v = s.read_prefix(0, 5)
    assert k.reshape(-1).tolist() == KEYS5.reshape(-1).tolist()
    assert v.reshape(-1).tolist() == VALS5.reshape(-1).tolist()
    infos = s.page_infos(0)
    assert [i[2] for i in infos] == [2, 2, 1, 0]


def test_paged_storage_prefix_handle_block_table(orc):
    # paged_kv.rs:969-1011
    s = orc.PagedKvStorage(1, 1, 2, 8, 2)
    s.write_sequence(0, 0, KEYS5, VALS5)
    assert s.block_table(0, 5) == [(0, 0, 0, 2), (1, 1, 2, 2), (2, 2, 4, 1)]


def test_paged_storage_imports_prefix(orc):
    # paged_kv.rs:1013-1068
    src = orc.PagedKvStorage(1, 1, 2, 8, 2)
    dst = orc.PagedKvStorage(1, 1, 2, 8, 2)
    src.write_sequence(0, 0, KEYS5, VALS5)
    dst.import_prefix_from(src, 5)
    k, v = dst.read_prefix(0, 5)
    assert k.reshape(-1).tolist() == KEYS5.reshape(-1).tolist()
    assert v.reshape(-1).tolist() == VALS5.reshape(-1).tolist()
    assert [i[2] for i in dst.page_infos(0)][:3] == [2, 2, 1]


def test_paged_storage_reuses_page_ids_after_reset(orc):
    # paged_kv.rs:1070-1113
    s = orc.PagedKvStorage(1, 1, 2, 8, 2)
    k = np.array([1, 2, 3, 4], np.float32).reshape(2, 1, 2)
    v = np.array([5, 6, 7, 8], np.float32).reshape(2, 1, 2)
    s.write_sequence(0, 0, k, v)
    assert s.allocated_pages(0) == 1 and s.free_pages(0) == 3
    s.reset()
    s.write_sequence(0, 2, k, v)
    infos = s.page_infos(0)
    assert s.allocated_pages(0) == 1 and s.free_pages(0) == 3
    assert infos[0] == (0, 2, 2)
    assert infos[1][2] == 0


def test_paged_storage_errors(orc):
    # paged_kv.rs:494-499 (pool exhausted), 865-882 (prefix length), 600-604 (capacity)
    s = orc.PagedKvStorage(1, 1, 2, 4, 2)
    with pytest.raises(orc.OracleError) as e:
        s.read_prefix(0, 0)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(orc.OracleError) as e:
        s.write_slot(0, 4, [[0, 0]], [[0, 0]])
    assert e.value.kind == "Runtime"
    with pytest.raises(orc.OracleError) as e:
        s.block_table(0, 2)  # nothing committed yet
    assert e.value.kind == "Runtime"


# ---- bf16 storage rule ----
def test_bf16_widening_and_rne(orc):
    # safetensors.rs:540-542: widening is bits << 16.  Narrowing (the GPU KV-append rule)
    # is round-to-nearest-even, checked on the tie / non-tie cases that separate it from
    # truncation (safetensors.rs:718-724 truncates in its test encoder).
    bits = np.array([0x3F80, 0xBF80, 0x4049, 0x0000, 0x8000], np.uint16)
    assert orc.bf16_to_f32(bits).tolist() == [1.0, -1.0, 3.140625, 0.0, -0.0]
    vals = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF], np.uint32).view(np.float32)
    assert orc.f32_to_bf16(vals).tolist() == [0x3F80, 0x3F82, 0x3F81, 0x3F80]


# ---- sampler (runtime/sampler.rs) ----
MASK64 = (1 << 64) - 1


def _xorshift_star(x):
    """One SamplerState::next_f32 step written from the published xorshift64* recurrence."""
    x ^= x >> 12
    x ^= (x << 25) & MASK64
    x ^= x >> 27
    value = (x * 0x2545F4914F6CDD1D) & MASK64
    return np.float32((value >> 40) / float(1 << 24)), x


def test_sampler_rng_matches_xorshift64_star(orc):
    assert orc.sampler_state_new(0) == 0x9E3779B97F4A7C15  # sampler.rs:57-61
    assert orc.sampler_state_new(123) == 123
    for seed in (0, 42, 123):
        st = orc.sampler_state_new(seed)
        x = st
        for _ in range(1000):
            v, st = orc.sampler_next_f32(st)
            want, x = _xorshift_star(x)
            assert st == x and np.float32(v) == want


def test_sampler_reference_unit_tests(orc):
    # sampler.rs:247-260: argmax of the last row [1, 3, 2] is 1
    tok, prob = orc.argmax_last_token(np.array([[0, 1, 2], [1, 3, 2]], np.float32))
    assert tok == 1 and 0.0 < prob <= 1.0
    # sampler.rs:262-284: top_k = 2 over [1, 3, 2, 0.5] samples 1 or 2
    tok, prob, _ = orc.sample_last_token(np.array([[1.0, 3.0, 2.0, 0.5]], np.float32), 1.0, 2, 1.0,
                                         orc.sampler_state_new(123))
    assert tok in (1, 2) and 0.0 < prob <= 1.0


def test_sampler_greedy_configs_take_argmax_and_keep_the_state(orc):
    row = np.array([[0.5, 2.0, 2.0, -1.0]], np.float32)  # ties: the last maximum (max_by)
    for t, k, p in ((0.0, 20, 0.9), (0.7, 1, 0.9), (0.7, 20, 0.0)):
        tok, prob, st = orc.sample_last_token(row, t, k, p, 77)
        assert (tok, prob) == orc.argmax_last_token(row) and tok == 2 and st == 77


def _draws(orc, row, t, k, p, n, seed=1):
    st = orc.sampler_state_new(seed)
    counts = np.zeros(row.shape[-1], np.int64)
    for _ in range(n):
        tok, _, st = orc.sample_last_token(row, t, k, p, st)
        counts[tok] += 1
    return counts


def test_sampler_frequencies_follow_the_weights(orc):
    row = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    n = 20000
    for t, k, keep in ((1.0, 4, [0, 1, 2, 3]), (0.5, 4, [0, 1, 2, 3]), (1.0, 2, [2, 3])):
        counts = _draws(orc, row, t, k, 1.0, n)
        w = np.zeros(4)
        w[keep] = np.exp(row[0, keep] / t)
        w /= w.sum()
        assert all(counts[i] == 0 for i in range(4) if i not in keep)
        sigma = np.sqrt(n * w * (1 - w)) + 1e-9
        assert np.all(np.abs(counts - n * w) <= 5 * sigma), (t, k, counts, n * w)


def test_sampler_top_p_keeps_the_shortest_reaching_prefix(orc):
    # sorted weights exp(l - 3): 1, e^-1, e^-2, e^-3 (total 1.553); top_p 0.7 -> cutoff 1.087:
    # the prefix {3, 2} is the first to reach it
    row = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    counts = _draws(orc, row, 1.0, 4, 0.7, 4000)
    assert counts[0] == 0 and counts[1] == 0 and counts[2] > 0 and counts[3] > 0
    counts = _draws(orc, row, 1.0, 4, 0.5, 500)  # 1 / 1.553 = 0.644 >= 0.5: only token 3
    assert counts[3] == 500


def test_sampler_top_k_replacement_order(orc):
    # sampler.rs:168-183: a full candidate list replaces its FIRST minimum (list order) only by
    # a strictly larger logit.  [1, 1, 5, 1], k = 2: (0,1),(1,1) -> 5 replaces position 0 ->
    # (2,5),(1,1); the last 1 is not larger -> candidates {2, 1}, never 0 or 3.
    counts = _draws(orc, np.array([[1.0, 1.0, 5.0, 1.0]], np.float32), 100.0, 2, 1.0, 400)
    assert counts[0] == 0 and counts[3] == 0 and counts[1] > 0 and counts[2] > 0
    # [3, 1, 1, 2], k = 2: the second 1 does not replace, 2 replaces the 1 at position 1 -> {0, 3}
    counts = _draws(orc, np.array([[3.0, 1.0, 1.0, 2.0]], np.float32), 100.0, 2, 1.0, 400)
    assert counts[1] == 0 and counts[2] == 0 and counts[0] > 0 and counts[3] > 0


def test_sampler_threshold_walk_and_stable_order(orc):
    # [2, 2, 0], k = V: stable sort keeps (0, 2) before (1, 2); weights 1, 1, e^-2 (T = 1);
    # threshold = u * total, subtracted in list order: token 0 iff u * total <= 1
    row = np.array([[2.0, 2.0, 0.0]], np.float32)
    st = orc.sampler_state_new(9)
    for _ in range(200):
        u, nxt = orc.sampler_next_f32(st)
        total = np.float32(1.0) + np.float32(1.0) + np.float32(np.exp(np.float32(-2.0)))
        thr = np.float32(np.float32(u) * total)
        want = 0 if thr - np.float32(1.0) <= 0 else (1 if thr - np.float32(1.0) - np.float32(1.0) <= 0 else 2)
        tok, prob, st = orc.sample_last_token(row, 1.0, 3, 1.0, st)
        assert st == nxt and tok == want
