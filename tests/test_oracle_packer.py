"""The oracle's batch packer over one global page pool (GlobalPagePacker), pinned before it is
used as the GPU runtime's packing oracle.

* A request that runs alone must get exactly the page ids, per logical block, that the
  reference's own per-session PagedKvCacheStorage assigns (paged_kv.rs:469-527, 794-796),
  whose block tables the golden tests already pin.
* With several requests, shared prefixes and chunked prefill the packing must satisfy what
  the paged layout requires: the slot of position p is table[p // bs] * bs + p % bs, slots are
  unique within a tick, a page that more than one live sequence references is never written,
  a copy-on-write entry moves exactly reused % bs rows, and every page returns to the pool.
"""
import numpy as np
import pytest

from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

BS = 16


def tiny_model(orc, layers=2, seed=0):
    cfg = dict(TINY_LLAMA_C1, layers=layers, hidden=64, heads=4, kv_heads=2, intermediate=96,
               vocab=512)
    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                      cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                      tie=cfg["tie"])
    model.set_weights(random_weights(cfg, seed=seed))
    return cfg, model


def check_tick(p):
    T = p["positions"].size
    B = p["context_lens"].size
    assert p["cu_seqlens"][0] == 0 and p["cu_seqlens"][-1] == T
    assert np.all(np.diff(p["cu_seqlens"]) > 0)
    for b in range(B):
        lo, hi = p["cu_seqlens"][b], p["cu_seqlens"][b + 1]
        pos = p["positions"][lo:hi]
        assert np.array_equal(pos, np.arange(p["context_lens"][b] - (hi - lo), p["context_lens"][b]))
        table = p["block_tables"][b]
        assert np.array_equal(p["slot_mapping"][lo:hi],
                              table[pos // BS].astype(np.int64) * BS + pos % BS)
    assert np.unique(p["slot_mapping"]).size == T


def test_single_request_matches_reference_page_assignment(orc):
    cfg, model = tiny_model(orc)
    sched = orc.Scheduler(model, page_size=BS, max_chunk=20, max_batch_tokens=20)
    sched.attach_packer(64, BS)
    seq = sched.submit(np.arange(45, dtype=np.uint32) % cfg["vocab"], max_new_tokens=6)
    compared = 0
    while sched.execute_next_tick() is not None:
        p = sched.packed()
        check_tick(p)
        ctx = int(p["context_lens"][0])
        for layer in range(cfg["layers"]):
            ref = sched.session_blocks(seq, layer, ctx)
            if ref is None:  # released in this tick
                continue
            assert list(p["block_tables"][0][: len(ref)]) == ref
            compared += 1
    assert compared >= 2 * 5
    assert sched.packer_free_pages() == 64


def test_pages_return_lifo_in_table_order(orc):
    """A finished sequence's pages go back in block-table order onto the LIFO list, so the next
    sequence takes them last-first."""
    cfg, model = tiny_model(orc, layers=1)
    sched = orc.Scheduler(model, page_size=BS)
    sched.attach_packer(8, BS)
    sched.submit(np.arange(40, dtype=np.uint32), max_new_tokens=1)
    while sched.execute_next_tick() is not None:
        pass
    assert sched.packer_free_pages() == 8
    sched.submit(np.arange(100, 140, dtype=np.uint32), max_new_tokens=1)
    sched.execute_next_tick()
    assert list(sched.packed()["block_tables"][0]) == [2, 1, 0]


@pytest.mark.parametrize("seed", [0, 1])
def test_shared_prefix_and_chunked_packing_invariants(orc, seed):
    cfg, model = tiny_model(orc, seed=seed)
    rng = np.random.default_rng(seed)
    base = rng.integers(0, cfg["vocab"], size=50).astype(np.uint32)
    reqs = [(base, 5),
            (np.concatenate([base[:37], rng.integers(0, 512, 9)]).astype(np.uint32), 4),
            (np.concatenate([base[:32], rng.integers(0, 512, 3)]).astype(np.uint32), 3),
            (base.copy(), 2),
            (rng.integers(0, 512, 23).astype(np.uint32), 6)]
    sched = orc.Scheduler(model, page_size=BS, max_batch=3, max_chunk=20, max_batch_tokens=50,
                          min_share=16)
    sched.attach_packer(256, BS)
    ids = [sched.submit(p, max_new_tokens=n) for p, n in reqs]
    live = {}  # sequence -> last packed block table
    copies = 0
    while True:
        t = sched.execute_next_tick()
        if t is None:
            break
        kind, updates = t
        p = sched.packed()
        check_tick(p)
        by_seq = {int(s): b for b, s in enumerate(p["sequence_ids"])}
        # copy-on-write entries: one per sharing update whose reuse ends inside a page
        expect = [u["reused"] % BS for u in updates if u["reused"] and u["reused"] % BS]
        assert list(p["copy_count"]) == expect
        copies += len(expect)
        # pages that two live sequences referenced before this tick are read-only now
        before = {}
        for s, table in live.items():
            for blk in table:
                before.setdefault(blk, set()).add(s)
        shared_before = {blk for blk, o in before.items() if len(o) > 1}
        written = set((p["slot_mapping"] // BS).tolist()) | set(p["copy_dst"].tolist())
        assert not (written & shared_before)
        reused = {u["sequence_id"]: u["reused"] for u in updates if u["reused"]}
        for s, b in by_seq.items():
            live[s] = list(p["block_tables"][b][: (p["context_lens"][b] + BS - 1) // BS])
        for s in reused:
            if s not in by_seq:  # shared its whole prompt, no rows of its own this tick
                live[s] = sched.packer_pages(s)
        # a row written this tick into a page that another sequence references is the row that
        # sequence sees at the same position: it shared the page in this tick, from the writer
        # (at a later point of the tick's order), up to at least this position
        for b, x in enumerate(int(v) for v in p["sequence_ids"]):
            lo, hi = p["cu_seqlens"][b], p["cu_seqlens"][b + 1]
            for pos, slot in zip(p["positions"][lo:hi], p["slot_mapping"][lo:hi]):
                page = int(slot) // BS
                for y, table in live.items():
                    if y == x or page not in table:
                        continue
                    assert y in reused and table.index(page) == pos // BS and pos < reused[y]
                    assert by_seq.get(y, len(by_seq)) > b
        for u in updates:
            if u["finish_reason"]:
                live.pop(u["sequence_id"], None)
    assert copies >= 1
    assert sched.packer_free_pages() == 256
    assert len(ids) == 5
