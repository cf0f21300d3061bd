"""Decode ticks replayed from HIP graphs (graph_decode) against eager execution and the oracle.

A graph replays the recorded launch sequence over the batch metadata re-uploaded into the same
buffers, with max_context_len rounded up to a 1024-token bucket.  Because every sequence's
reduction order depends only on its own context length, replayed ticks must reproduce the eager
ticks bit for bit: same tick log, same tokens, same probabilities (and, for a sampler, the same
device-advanced states).  Each run performs many replays separated by the runtime's own eager
work (prefill ticks, metadata uploads, downloads and fault checks), and every replayed tick's
output is compared.  The graph runs are also held to the oracle like the eager runtime
(tests/test_gpu_model.py::compare).
"""
import numpy as np
import pytest

from test_gpu_model import compare, drive

pytestmark = pytest.mark.gpu


def make_runtime(cfg, weights, graph, sched_kw, num_blocks=4096, sampler=None, weight_dtype="f32",
                 kv_dtype="f32"):
    from ferrisinfer_amd.runtime import Runtime

    rt = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                 cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"], tie=cfg["tie"],
                 num_blocks=num_blocks, block_size=16, sampler=sampler, graph_decode=graph,
                 weight_dtype=weight_dtype, kv_dtype=kv_dtype, **sched_kw)
    rt.set_weights(weights)
    return rt


def oracle_scheduler(orc, cfg, weights, sched_kw, num_blocks=4096):
    """The oracle's reference scheduler with the global page packer, as build_pair makes it."""
    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                      cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                      tie=cfg["tie"])
    model.set_weights(weights)
    ref = orc.Scheduler(model, page_size=16, **sched_kw)
    ref.attach_packer(num_blocks, 16)
    return model, ref


def assert_same_run(eager, graph, requests):
    eid, eticks = drive(eager, requests)
    gid, gticks = drive(graph, requests)
    assert eid == gid and len(eticks) == len(gticks)
    for t, ((ek, eu), (gk, gu)) in enumerate(zip(eticks, gticks)):
        assert ek == gk, t
        for a, b in zip(eu, gu):
            for key in ("sequence_id", "reused", "appended", "phase", "finish_reason", "token",
                        "released"):
                assert a[key] == b[key], (t, key, a, b)
            if a["token"] is not None:
                # bit-identical probabilities: the replay ran the eager kernels on the same data
                assert np.float32(a["probability"]) == np.float32(b["probability"]), (t, a, b)
    for seq in eid:
        assert eager.generated(seq) == graph.generated(seq)
    return gticks


def test_graph_decode_matches_eager_and_reference(orc):
    """C1 (tiny Llama) requests, then a prefix-sharing set with chunked prefill and copy-on-write
    between the replays: the graph runtime against the eager runtime (bit-exact) and against the
    oracle scheduler (the runtime's parity bar)."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    print("graph decode: C1 + sharing", flush=True)
    cfg = TINY_LLAMA_C1
    weights = random_weights(cfg, seed=0)
    requests = c1_requests(0)
    eager = make_runtime(cfg, weights, False, {})
    graph = make_runtime(cfg, weights, True, {})
    assert_same_run(eager, graph, requests)
    c = graph.graph_counters()
    print(f"graph counters {c}", flush=True)
    assert c["replays"] > 20 and c["captures"] >= 1
    assert graph.pool_free_count() == 4096
    # the graph runtime against the oracle, with the same comparison as the eager one
    model, ref = oracle_scheduler(orc, cfg, weights, {})
    _, ties = compare(model, ref, make_runtime(cfg, weights, True, {}), requests)
    assert ties == 0
    rng = np.random.default_rng(7)
    base = rng.integers(0, cfg["vocab"], size=40).astype(np.uint32)
    sharing = [
        (base.copy(), 6),
        (np.concatenate([base[:37], rng.integers(0, 4096, 9)]).astype(np.uint32), 5),
        (base.copy(), 3),
        (rng.integers(0, 4096, 23).astype(np.uint32), 7),
    ]
    kw = dict(max_batch=3, max_chunk=20, max_batch_tokens=50, min_share=16)
    assert_same_run(make_runtime(cfg, weights, False, kw), make_runtime(cfg, weights, True, kw), sharing)
    model, ref = oracle_scheduler(orc, cfg, weights, kw)
    compare(model, ref, make_runtime(cfg, weights, True, kw), sharing)


def test_graph_decode_across_context_buckets(orc):
    """Contexts that cross the 1024-token bucket (prompts of 990-1010 tokens, 40 new tokens):
    a new graph per bucket, identical to eager, oracle tokens."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    print("graph decode: crossing the 1024 bucket", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=4)
    rng = np.random.default_rng(12)
    requests = [(rng.integers(0, cfg["vocab"], n).astype(np.uint32), 40) for n in (990, 1001, 1010)]
    kw = dict(max_chunk=512, max_batch_tokens=2048)
    eager = make_runtime(cfg, weights, False, kw)
    graph = make_runtime(cfg, weights, True, kw)
    assert_same_run(eager, graph, requests)
    c = graph.graph_counters()
    print(f"graph counters {c}", flush=True)
    assert c["captures"] >= 2 and c["replays"] > 30
    model, ref = oracle_scheduler(orc, cfg, weights, kw)
    compare(model, ref, make_runtime(cfg, weights, True, kw), requests)


@pytest.mark.parametrize("sampler", [(0.8, 20, 0.9, 42), (0.9, 3000, 0.95, 7)])
def test_graph_decode_sampled_matches_eager(orc, sampler):
    """The device sampler inside the replayed tick: per-row states are uploaded before and read
    back after every replay; tokens, probabilities and the tick log equal the eager run's.  Top-k
    3000 puts the reserved-area sampling launch in the graphs."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    print(f"graph decode sampled {sampler}", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=3, std=0.05)
    eager = make_runtime(cfg, weights, False, {}, sampler=sampler)
    graph = make_runtime(cfg, weights, True, {}, sampler=sampler)
    assert_same_run(eager, graph, c1_requests(0))
    assert graph.graph_counters()["replays"] > 20


def test_graph_decode_c4_shape_batch_64():
    """The C4 model shape at decode batch 64 (64 requests, 32-token prompts, 8 new tokens):
    replayed ticks identical to eager ones."""
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, random_weights

    print("graph decode: C4 shape batch 64", flush=True)
    cfg = QWEN2_05B_C4
    weights = random_weights(cfg, seed=0, qkv_bias=True)
    rng = np.random.default_rng(64)
    requests = [(rng.integers(0, cfg["vocab"], 32).astype(np.uint32), 8) for _ in range(64)]
    kw = dict(max_batch=64, max_seq=64)
    eager = make_runtime(cfg, weights, False, kw, num_blocks=512)
    graph = make_runtime(cfg, weights, True, kw, num_blocks=512)
    del weights
    gticks = assert_same_run(eager, graph, requests)
    assert sum(1 for kind, us in gticks if kind == 1 and len(us) == 64) >= 7
    assert graph.graph_counters()["replays"] >= 5
