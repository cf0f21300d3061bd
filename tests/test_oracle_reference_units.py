"""The reference's own unit tests for the host-side integer logic, run against the oracle.

Each test below restates one `#[test]` of the reference's runtime crate with the same inputs
and the same assertions (file:line in each docstring), so the oracle's restatement of the
scheduler, prefix index, prefix block manager, sequence state, session and KV cache is pinned
by the reference's expectations rather than by a second restatement.  The fixtures are the
reference's: `always_one_model` (scheduler.rs:1323-1409, session.rs:647-718) — hidden 1, every
projection 0, output weight [[0], [1]], so every sampled token is 1 — and the a->0 / b->1
dummy tokenizer (session.rs:436-486), whose encode/decode the tests apply by hand.

The GPU runtime's scheduler is compared tick by tick with this oracle in
tests/test_gpu_model.py; pinning the oracle here closes that chain.
"""
import numpy as np
import pytest

import oracle
from oracle import (FINISH_REASONS, PHASES, KvCache, PrefixBlockManager, PrefixIndex, SequenceState,
                    scheduler_plan_next_tick, scheduler_resident_session_count,
                    scheduler_sequence_state, scheduler_shared_prefix_source, session_generate_from_tokens,
                    session_kv_is_paged, session_kv_used_tokens, session_prefix_handle,
                    session_token_history)

PREFILL, DECODE = 0, 1


# ----------------------------------------------------------------------------- fixtures
def always_one_model():
    """scheduler.rs:1323-1409: a 1-layer, hidden-1 Qwen2-shaped model whose logits always pick
    token 1 (every projection 0, output weight [[0], [1]], rotary_dims 0)."""
    m = oracle.Model(hidden=1, intermediate=1, layers=1, heads=1, kv_heads=1, vocab=2, max_pos=16,
                     eps=1e-6, theta=10000.0, rotary_dims=0, tie=False)
    one = np.ones(1, np.float32)
    zero = np.zeros((1, 1), np.float32)
    m.set_weights({
        "tok_embeddings.weight": np.ones((2, 1), np.float32),
        "layers.0.attention_norm.weight": one,
        "layers.0.attention.wq.weight": zero,
        "layers.0.attention.wk.weight": zero,
        "layers.0.attention.wv.weight": zero,
        "layers.0.attention.wo.weight": zero,
        "layers.0.ffn_norm.weight": one,
        "layers.0.feed_forward.w1.weight": zero,
        "layers.0.feed_forward.w2.weight": zero,
        "layers.0.feed_forward.w3.weight": zero,
        "norm.weight": one,
        "output.weight": np.array([[0.0], [1.0]], np.float32),
    })
    return m


def encode(text):
    """DummyTokenizer::encode without BOS (session.rs:448-468)."""
    return [{"a": 0, "A": 0, "b": 1, "B": 1}[c] for c in text]


def decode(tokens):
    """DummyTokenizer::decode (session.rs:470-485)."""
    return "".join({0: "A", 1: "B"}[t] for t in tokens)


def make_scheduler(page_size=0, max_seq=4096, max_gen=512, **cfg):
    """test_scheduler (scheduler.rs:1311-1321) with SessionConfig / SchedulerConfig overrides;
    page_size 0 = SessionKvCacheConfig::Contiguous (the default)."""
    keys = dict(max_batch_size="max_batch", max_prefill_chunk_tokens="max_chunk",
                max_prefill_batch_tokens="max_batch_tokens",
                max_consecutive_prefill_ticks="max_consecutive_prefill",
                min_prefix_share_tokens="min_share")
    kw = {keys[k]: v for k, v in cfg.items()}
    model = always_one_model()
    s = oracle.Scheduler(model, max_seq=max_seq, max_gen=max_gen, page_size=page_size, **kw)
    s._model = model
    return s


def tick(s):
    kind, updates = s.execute_next_tick()
    for u in updates:
        u["phase"] = PHASES[u["phase"]]
        u["finish_reason"] = FINISH_REASONS[u["finish_reason"]]
    return kind, updates


# ----------------------------------------------------------------------------- scheduler.rs
def test_reference_scheduler_prefills_then_decodes_single_sequence():
    """scheduler.rs:720-765."""
    s = make_scheduler()
    seq = s.submit([0, 1], max_new_tokens=1)
    assert scheduler_plan_next_tick(s) == ("Prefill", [seq])
    kind, up = tick(s)
    assert kind == PREFILL
    assert up[0]["reused"] == 0 and up[0]["appended"] == 2
    assert up[0]["token"] is None
    assert up[0]["phase"] == "Decode" and up[0]["finish_reason"] is None
    kind, up = tick(s)
    assert kind == DECODE
    assert up[0]["sequence_id"] == seq and up[0]["token"] == 1
    assert up[0]["finish_reason"] == "MaxNewTokens"
    st = scheduler_sequence_state(s, seq)
    assert st["phase"] == "Finished" and st["finish_reason"] == "MaxNewTokens"
    assert s.generated(seq) == [1]
    assert s.execute_next_tick() is None


def test_reference_scheduler_prefill_has_priority_over_decode():
    """scheduler.rs:768-804."""
    s = make_scheduler(max_batch_size=1)
    first = s.submit([0], max_new_tokens=2)
    tick(s)
    assert scheduler_plan_next_tick(s)[0] == "Decode"
    second = s.submit([1], max_new_tokens=1)
    assert scheduler_plan_next_tick(s) == ("Prefill", [second])
    assert scheduler_sequence_state(s, first)["phase"] == "Decode"


def test_reference_scheduler_chunked_prefill_spreads_prompt_across_ticks():
    """scheduler.rs:807-849."""
    s = make_scheduler(max_batch_size=1, max_prefill_chunk_tokens=2)
    seq = s.submit([0, 1, 0, 1, 0], max_new_tokens=1)
    for appended, phase in ((2, "Prefill"), (2, "Prefill"), (1, "Decode")):
        kind, up = tick(s)
        assert kind == PREFILL
        assert up[0]["appended"] == appended and up[0]["phase"] == phase
    kind, up = tick(s)
    assert kind == DECODE and up[0]["token"] == 1
    assert scheduler_sequence_state(s, seq)["finish_reason"] == "MaxNewTokens"


def test_reference_scheduler_reuses_prompt_prefix_from_existing_sequence():
    """scheduler.rs:852-892: reused 3 (the 4-token prompts share [0, 1, 0]), appended 1."""
    s = make_scheduler(page_size=2, max_batch_size=1, min_prefix_share_tokens=2)
    first = s.submit([0, 1, 0, 1], max_new_tokens=1)
    tick(s)
    second = s.submit([0, 1, 0, 0], max_new_tokens=1)
    kind, up = tick(s)
    assert kind == PREFILL
    assert [u["sequence_id"] for u in up] == [second]
    assert up[0]["reused"] == 3 and up[0]["appended"] == 1
    assert up[0]["phase"] == "Decode"
    assert scheduler_sequence_state(s, first)["phase"] == "Decode"


def test_reference_scheduler_tracks_shared_prefix_block_metadata():
    """scheduler.rs:895-941: both of the source's blocks are referenced twice."""
    s = make_scheduler(page_size=2, max_batch_size=1, min_prefix_share_tokens=2)
    first = s.submit([0, 1, 0, 1], max_new_tokens=1)
    tick(s)
    second = s.submit([0, 1, 0, 0], max_new_tokens=1)
    tick(s)
    assert s.block_ref_count(first, 0, 0) == 2
    assert s.block_ref_count(first, 0, 1) == 2
    assert scheduler_shared_prefix_source(s, second) == first


def test_reference_scheduler_releases_finished_paged_sequence_resources():
    """scheduler.rs:944-981: the finished sequence's one block is released, in the report."""
    s = make_scheduler(page_size=2)
    seq = s.submit([0, 1], max_new_tokens=1)
    assert scheduler_resident_session_count(s) == 1
    _, up = tick(s)
    assert up[0]["released"] == []
    _, up = tick(s)
    assert up[0]["finish_reason"] == "MaxNewTokens"
    assert scheduler_resident_session_count(s) == 0
    assert s.block_ref_count(seq, 0, 0) == 0
    assert up[0]["released"] == [(seq, 0, 0)]


def test_reference_scheduler_releases_shared_prefix_refs_when_target_finishes():
    """scheduler.rs:984-1039."""
    s = make_scheduler(page_size=2, max_batch_size=2, min_prefix_share_tokens=2)
    first = s.submit([0, 1, 0, 1], max_new_tokens=3)
    tick(s)
    second = s.submit([0, 1, 0, 0], max_new_tokens=1)
    tick(s)
    _, up = tick(s)
    su = next(u for u in up if u["sequence_id"] == second)
    assert su["finish_reason"] == "MaxNewTokens"
    assert scheduler_resident_session_count(s) == 1
    assert s.block_ref_count(first, 0, 0) == 1
    assert s.block_ref_count(first, 0, 1) == 1
    assert su["released"] != []


def test_reference_scheduler_does_not_reuse_full_prompt_after_source_has_decoded():
    """scheduler.rs:1042-1076: an identical 3-token prompt reuses 2, not 3."""
    s = make_scheduler(page_size=2, max_batch_size=1, min_prefix_share_tokens=2)
    s.submit([0, 1, 0], max_new_tokens=2)
    tick(s)
    tick(s)
    second = s.submit([0, 1, 0], max_new_tokens=1)
    _, up = tick(s)
    assert up[0]["sequence_id"] == second
    assert up[0]["reused"] == 2 and up[0]["appended"] == 1


def test_reference_scheduler_breaks_prefill_streak_with_decode_when_decode_is_waiting():
    """scheduler.rs:1079-1120."""
    s = make_scheduler(max_batch_size=1, max_prefill_chunk_tokens=2, max_consecutive_prefill_ticks=2)
    first = s.submit([0, 1, 0, 1], max_new_tokens=2)
    tick(s)
    tick(s)
    second = s.submit([1, 0, 1, 0], max_new_tokens=1)
    assert scheduler_plan_next_tick(s) == ("Decode", [first])
    kind, up = tick(s)
    assert kind == DECODE
    assert up[0]["sequence_id"] == first and up[0]["token"] == 1
    assert scheduler_sequence_state(s, second)["phase"] == "Prefill"


def test_reference_scheduler_prefill_batch_respects_token_budget_and_packs_remainder_chunks():
    """scheduler.rs:1123-1156: 4 + 4 tokens exceed the budget of 5; the 1-token remainder packs
    with the second sequence's chunk."""
    s = make_scheduler(max_batch_size=4, max_prefill_chunk_tokens=4, max_prefill_batch_tokens=5)
    first = s.submit([0, 1, 0, 1, 0], max_new_tokens=1)
    second = s.submit([1, 0, 1, 0], max_new_tokens=1)
    assert scheduler_plan_next_tick(s) == ("Prefill", [first])
    tick(s)
    assert scheduler_plan_next_tick(s) == ("Prefill", [first, second])


def test_reference_scheduler_prefers_full_decode_batch_between_prefill_chunks():
    """scheduler.rs:1159-1206."""
    s = make_scheduler(max_batch_size=2, max_prefill_chunk_tokens=2, max_consecutive_prefill_ticks=8)
    first = s.submit([0], max_new_tokens=2)
    tick(s)
    second = s.submit([1], max_new_tokens=2)
    tick(s)
    third = s.submit([0, 1, 0, 1], max_new_tokens=1)
    assert scheduler_plan_next_tick(s) == ("Decode", [first, second])
    kind, up = tick(s)
    assert kind == DECODE and [u["sequence_id"] for u in up] == [first, second]
    assert scheduler_sequence_state(s, third)["phase"] == "Prefill"


def test_reference_scheduler_decode_tick_batches_multiple_sequences_after_staggered_prefill():
    """scheduler.rs:1209-1249."""
    s = make_scheduler(max_batch_size=2)
    first = s.submit([0], max_new_tokens=1)
    tick(s)
    second = s.submit([1], max_new_tokens=1)
    tick(s)
    kind, up = tick(s)
    assert kind == DECODE and [u["sequence_id"] for u in up] == [first, second]
    assert len(up) == 2
    assert all(u["token"] is not None for u in up)
    assert all(u["finish_reason"] == "MaxNewTokens" for u in up)


def test_reference_scheduler_reports_session_limit_finish_reason():
    """scheduler.rs:1252-1284: requested 3 > session budget 1 -> SessionLimit."""
    s = make_scheduler(max_seq=8, max_gen=1)
    seq = s.submit([0], max_new_tokens=3)
    tick(s)
    _, up = tick(s)
    assert up[0]["finish_reason"] == "SessionLimit"
    assert scheduler_sequence_state(s, seq)["finish_reason"] == "SessionLimit"


def test_reference_scheduler_can_finish_immediately_after_prefill():
    """scheduler.rs:1287-1309."""
    s = make_scheduler()
    seq = s.submit([0], max_new_tokens=0)
    kind, up = tick(s)
    assert kind == PREFILL
    assert up[0]["finish_reason"] == "MaxNewTokens"
    assert scheduler_sequence_state(s, seq)["phase"] == "Finished"


# ----------------------------------------------------------------------------- prefix_index.rs
def test_prefix_index_groups_candidates_by_minimum_prefix_bucket():
    """prefix_index.rs:115-143."""
    index = PrefixIndex(2)
    index.upsert(1, [10, 11, 12, 13], 4, 4)
    index.upsert(2, [10, 11, 99], 3, 3)
    index.upsert(3, [10, 12, 13], 3, 3)
    assert index.best_match(7, [10, 11, 12, 99]) == (1, 3)


def test_prefix_index_avoids_full_prompt_share_when_source_has_decode_token():
    """prefix_index.rs:146-160."""
    index = PrefixIndex(2)
    index.upsert(1, [1, 2, 3], 3, 4)
    assert index.best_match(9, [1, 2, 3]) == (1, 2)


# ----------------------------------------------------------------------------- block_manager.rs
def _handle(token_count, page_size, entries):
    """PrefixHandle::new_for_tests over one layer of KvBlockTableEntry::new_for_tests
    (logical index, block id, start, count)."""
    return {"token_count": token_count, "page_size": page_size, "layers": [entries]}


def test_prefix_block_manager_updates_owned_prefix_ref_counts():
    """block_manager.rs:180-216."""
    m = PrefixBlockManager()
    full = _handle(4, 2, [(0, 0, 0, 2), (1, 1, 2, 2)])
    shorter = _handle(2, 2, [(0, 0, 0, 2)])
    m.update_owned_prefix(3, full)
    assert m.block_ref_count(3, 0, 0) == 1
    assert m.block_ref_count(3, 0, 1) == 1
    m.update_owned_prefix(3, shorter)
    assert m.block_ref_count(3, 0, 0) == 1
    assert m.block_ref_count(3, 0, 1) == 0


def test_prefix_block_manager_tracks_shared_prefix_references_against_source_blocks():
    """block_manager.rs:219-276."""
    m = PrefixBlockManager()
    shared = _handle(3, 2, [(0, 0, 0, 2), (1, 1, 2, 1)])
    m.update_owned_prefix(1, shared)
    m.update_shared_prefix(2, (1, shared))
    assert m.block_ref_count(1, 0, 0) == 2
    assert m.block_ref_count(1, 0, 1) == 2
    assert m.remove_sequence(2) == []
    assert m.block_ref_count(1, 0, 0) == 1
    assert m.block_ref_count(1, 0, 1) == 1


def test_prefix_block_manager_reports_released_blocks_when_owner_is_removed():
    """block_manager.rs:279-304: released in block-table order."""
    m = PrefixBlockManager()
    m.update_owned_prefix(7, _handle(4, 2, [(0, 0, 0, 2), (1, 1, 2, 2)]))
    released = m.remove_sequence(7)
    assert m.tracked_block_count() == 0
    assert released == [(7, 0, 0), (7, 0, 1)]


# ----------------------------------------------------------------------------- sequence.rs
def test_sequence_state_tracks_prefill_decode_and_finish():
    """sequence.rs:244-287."""
    s = SequenceState(7, 11, [1, 2, 3], 16, stop_token_id=99)
    st = s.state()
    assert st["request_id"] == 7 and st["sequence_id"] == 11
    assert st["prompt_len"] == 3 and s.generated_tokens() == [] and st["generated_len"] == 0
    assert st["cached_tokens"] == 0 and st["cached_prompt_tokens"] == 0
    assert st["pending_prompt_tokens"] == 3
    assert st["requested_max_new_tokens"] == 16 and st["max_new_tokens"] == 16
    assert st["stop_token_id"] == 99
    assert st["phase"] == "Prefill" and st["finish_reason"] is None
    assert not st["is_finished"] and not st["generation_budget_reached"]
    s.record_prefill(3)
    st = s.state()
    assert st["cached_tokens"] == 3 and st["cached_prompt_tokens"] == 3
    assert st["pending_prompt_tokens"] == 0 and st["phase"] == "Decode"
    s.record_generated_token(42)
    st = s.state()
    assert s.generated_tokens() == [42] and st["generated_len"] == 1
    assert st["cached_tokens"] == 4 and st["total_tokens"] == 4
    s.finish("StopToken")
    st = s.state()
    assert st["phase"] == "Finished" and st["finish_reason"] == "StopToken" and st["is_finished"]


def test_sequence_state_stays_in_prefill_until_prompt_is_fully_cached():
    """sequence.rs:290-318."""
    s = SequenceState(3, 5, [10, 11, 12, 13, 14], 8)
    assert s.next_prefill_chunk(2) == [10, 11]
    s.record_prefill(2)
    st = s.state()
    assert (st["cached_prompt_tokens"], st["pending_prompt_tokens"], st["phase"]) == (2, 3, "Prefill")
    assert s.next_prefill_chunk(2) == [12, 13]
    s.record_prefill(2)
    st = s.state()
    assert (st["cached_prompt_tokens"], st["pending_prompt_tokens"], st["phase"]) == (4, 1, "Prefill")
    assert s.next_prefill_chunk(2) == [14]
    s.record_prefill(1)
    st = s.state()
    assert (st["cached_prompt_tokens"], st["pending_prompt_tokens"], st["phase"]) == (5, 0, "Decode")


def test_sequence_state_distinguishes_requested_limit_from_session_budget():
    """sequence.rs:321-342."""
    s = SequenceState(1, 2, [7], 4, generation_budget=1)
    st = s.state()
    assert st["requested_max_new_tokens"] == 4 and st["max_new_tokens"] == 1
    assert st["generation_budget_finish_reason"] == "SessionLimit"
    s.record_prefill(1)
    s.record_generated_token(99)
    assert s.state()["generation_budget_reached"]


def test_scheduler_tick_reports_batch_shape():
    """sequence.rs:345-356, on a tick the oracle scheduler plans: two decode-phase sequences
    form one Decode tick listing both ids in order."""
    s = make_scheduler(max_batch_size=2)
    a = s.submit([0], max_new_tokens=4)
    b = s.submit([1], max_new_tokens=4)
    tick(s)
    kind, ids = scheduler_plan_next_tick(s)
    assert kind == "Decode" and ids == [a, b] and len(ids) > 0


# ----------------------------------------------------------------------------- session.rs
def make_session(page_size=0, max_seq=4096, max_gen=512):
    model = always_one_model()
    s = oracle.Session(model, max_seq=max_seq, max_gen=max_gen, page_size=page_size)
    s._model = model
    return s


def test_prefill_tokens_tracks_history_and_cache_usage():
    """session.rs:490-498."""
    s = make_session()
    s.prefill([0])
    assert s.position == 1 and session_kv_used_tokens(s) == 1
    assert session_token_history(s) == [0]


def test_prefill_tokens_batches_initial_prompt_and_preserves_last_sample():
    """session.rs:501-510."""
    s = make_session()
    s.prefill([0, 1])
    token, _ = s.step()
    assert s.position == 3 and session_kv_used_tokens(s) == 3
    assert session_token_history(s) == [0, 1, 1] and token == 1


def test_prefill_tokens_batches_appended_prompt_and_preserves_last_sample():
    """session.rs:513-524."""
    s = make_session()
    s.prefill([0])
    s.prefill([1, 0])
    token, _ = s.step()
    assert s.position == 4 and session_kv_used_tokens(s) == 4
    assert session_token_history(s) == [0, 1, 0, 1] and token == 1


def test_paged_kv_cache_prefill_and_decode_remain_functional():
    """session.rs:527-544."""
    s = make_session(page_size=2)
    s.prefill([0, 1, 0])
    token, _ = s.step()
    assert session_kv_is_paged(s)
    assert s.position == 4 and session_kv_used_tokens(s) == 4
    assert session_token_history(s) == [0, 1, 0, 1] and token == 1


def test_paged_session_exposes_prefix_handle():
    """session.rs:547-559."""
    s = make_session(page_size=2)
    s.prefill([0, 1, 0])
    h = session_prefix_handle(s, 3)
    assert h["token_count"] == 3 and h["page_size"] == 2 and len(h["layers"][0]) == 2


def test_copy_prefix_from_session_preserves_decode_state_for_exact_prefix():
    """session.rs:562-581: the destination continues from the source's last sample."""
    model = always_one_model()
    source = oracle.Session(model, page_size=2)
    dest = oracle.Session(model, page_size=2)
    source.prefill([0, 1, 0])
    dest.copy_prefix_from(source, 3)
    token, _ = dest.step()
    assert dest.position == 4 and session_kv_used_tokens(dest) == 4
    assert session_token_history(dest) == [0, 1, 0, 1] and token == 1


def test_generate_reference_from_tokens_stops_on_stop_token():
    """session.rs:584-597."""
    s = make_session()
    samples, finish = session_generate_from_tokens(s, [0], 4, stop_token_id=1)
    assert [t for t, _ in samples] == [1] and decode([t for t, _ in samples]) == "B"
    assert finish == "StopToken"
    assert session_token_history(s) == [0, 1] and session_kv_used_tokens(s) == 2


def test_generate_reference_respects_session_generation_limit():
    """session.rs:600-619: the prompt "a" without BOS encodes to [0]."""
    s = make_session(max_seq=8, max_gen=1)
    prompt = encode("a")
    assert prompt == [0]
    samples, finish = session_generate_from_tokens(s, prompt, 3)
    assert [t for t, _ in samples] == [1] and decode([t for t, _ in samples]) == "B"
    assert finish == "SessionLimit"


# ----------------------------------------------------------------------------- kv_cache.rs
def test_contiguous_storage_implements_storage_trait():
    """kv_cache.rs:675-692: one layer of key storage [8, 1, 2]."""
    c = KvCache(1, 1, 2, 8).counts()
    assert not c["paged"] and c["layers"] == 1 and c["layer_elements"] == 8 * 1 * 2


def test_kv_cache_allocates_layer_storage():
    """kv_cache.rs:695-709."""
    c = KvCache(2, 1, 2, 8).counts()
    assert not c["paged"] and c["layers"] == 2 and c["layer_elements"] == 8 * 1 * 2


def test_kv_cache_write_and_read_prefix_round_trip():
    """kv_cache.rs:712-744."""
    cache = KvCache(1, 1, 2, 8)
    first, second = cache.reserve_slot(), cache.reserve_slot()
    assert (first, second) == (0, 1)
    cache.write(0, first, [1.0, 2.0], [3.0, 4.0])
    cache.write(0, second, [5.0, 6.0], [7.0, 8.0])
    k, v = cache.read_prefix(0, 2)
    assert k.shape == (2, 1, 2) and v.shape == (2, 1, 2)
    assert k.reshape(-1).tolist() == [1.0, 2.0, 5.0, 6.0]
    assert v.reshape(-1).tolist() == [3.0, 4.0, 7.0, 8.0]


def test_kv_cache_reset_restores_capacity():
    """kv_cache.rs:747-764."""
    cache = KvCache(1, 1, 2, 8)
    cache.advance(3)
    c = cache.counts()
    assert (c["used_tokens"], c["remaining_tokens"]) == (3, 5)
    cache.reset()
    c = cache.counts()
    assert (c["used_tokens"], c["remaining_tokens"]) == (0, 8)


def test_kv_cache_write_sequence_uncommitted_round_trip():
    """kv_cache.rs:767-796."""
    cache = KvCache(1, 1, 2, 8)
    cache.write_sequence_uncommitted(0, 0, [[[1.0, 2.0]], [[5.0, 6.0]]], [[[3.0, 4.0]], [[7.0, 8.0]]])
    cache.advance(2)
    k, v = cache.read_prefix(0, 2)
    assert k.reshape(-1).tolist() == [1.0, 2.0, 5.0, 6.0]
    assert v.reshape(-1).tolist() == [3.0, 4.0, 7.0, 8.0]


KEYS3 = [[[1.0, 2.0]], [[5.0, 6.0]], [[9.0, 10.0]]]
VALS3 = [[[3.0, 4.0]], [[7.0, 8.0]], [[11.0, 12.0]]]


def test_paged_kv_cache_exposes_prefix_handle():
    """kv_cache.rs:799-832."""
    cache = KvCache(1, 1, 2, 8, page_size=2)
    cache.write_sequence_uncommitted(0, 0, KEYS3, VALS3)
    cache.advance(3)
    h = cache.prefix_handle(3)
    assert h["token_count"] == 3 and h["page_size"] == 2 and len(h["layers"][0]) == 2


def test_paged_kv_cache_copy_prefix_from_round_trip():
    """kv_cache.rs:835-888."""
    source = KvCache(1, 1, 2, 8, page_size=2)
    dest = KvCache(1, 1, 2, 8, page_size=2)
    source.write_sequence_uncommitted(0, 0, KEYS3, VALS3)
    source.advance(3)
    dest.copy_prefix_from(source, 3)
    k, v = dest.read_prefix(0, 3)
    c = dest.counts()
    assert c["paged"] and c["used_tokens"] == 3
    assert k.reshape(-1).tolist() == [1.0, 2.0, 5.0, 6.0, 9.0, 10.0]
    assert v.reshape(-1).tolist() == [3.0, 4.0, 7.0, 8.0, 11.0, 12.0]


def test_kv_cache_copy_prefix_from_falls_back_across_storage_kinds():
    """kv_cache.rs:891-933: contiguous source, paged destination."""
    source = KvCache(1, 1, 2, 8)
    dest = KvCache(1, 1, 2, 8, page_size=2)
    source.write_sequence_uncommitted(0, 0, KEYS3[:2], VALS3[:2])
    source.advance(2)
    dest.copy_prefix_from(source, 2)
    k, v = dest.read_prefix(0, 2)
    assert dest.counts()["used_tokens"] == 2
    assert k.reshape(-1).tolist() == [1.0, 2.0, 5.0, 6.0]
    assert v.reshape(-1).tolist() == [3.0, 4.0, 7.0, 8.0]


def test_kv_cache_rejects_writes_outside_the_commit_protocol():
    """kv_cache.rs:441-471, 584-594: a committed write needs a reserved position; an uncommitted
    write may not skip past the next slot; a read may not pass the committed tokens."""
    cache = KvCache(1, 1, 2, 8)
    with pytest.raises(oracle.OracleError) as e:
        cache.write(0, 0, [1.0, 2.0], [3.0, 4.0])
    assert e.value.kind == "InvalidShape"
    with pytest.raises(oracle.OracleError) as e:
        cache.write_uncommitted(0, 1, [1.0, 2.0], [3.0, 4.0])
    assert e.value.kind == "InvalidShape"
    cache.write_uncommitted(0, 0, [1.0, 2.0], [3.0, 4.0])
    with pytest.raises(oracle.OracleError) as e:
        cache.read_prefix(0, 1)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(oracle.OracleError) as e:
        cache.advance(9)
    assert e.value.kind == "Runtime"
