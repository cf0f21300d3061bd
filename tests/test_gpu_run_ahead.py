"""Decode ticks enqueued ahead (FR_TICK_RUN_AHEAD) against ticks run one call at a time.

With run_ahead, a call that enqueues a tick also enqueues the next one when that will be a
greedy decode tick: its batch follows from the state the tick leaves, and its token ids are
the tick's samples, fed on the device.  The next call keeps it when its own planning packs the
same batch and drops it otherwise (a submit in between).  Every test compares the whole run
with a runtime driven without the flag:
  * tick kinds and every update (tokens, probability bits, finish reasons, released blocks);
  * after every tick, the pool's free count and each sequence's block list.
Each test also checks that ticks were kept, and dropped where submits interleave.  The
serial runtime is held to the oracle by tests/test_gpu_model.py; one test here holds the
run-ahead runtime to the oracle directly.
"""
import numpy as np
import pytest

from test_gpu_graph import make_runtime, oracle_scheduler
from test_gpu_model import compare

pytestmark = pytest.mark.gpu


def drive(rt, requests, mode):
    """requests: (prompt, max_new, stop, arrival_tick), submitted before the tick of their
    arrival.  mode: None (no flag), "always" (the flag on every call, also before a submit,
    which drops the enqueued tick) or "quiet" (the flag when no request arrives before the next
    call)."""
    order = sorted(range(len(requests)), key=lambda i: requests[i][3])
    ids = [None] * len(requests)  # sequence id of each request, in request order
    log, snaps = [], []
    nxt, tick = 0, 0
    while True:
        while nxt < len(order) and requests[order[nxt]][3] <= tick:
            prompt, n, stop, _ = requests[order[nxt]]
            ids[order[nxt]] = rt.submit(prompt, max_new_tokens=n, stop_token=stop)
            nxt += 1
        if mode is None:
            rep = rt.execute_next_tick()
        else:
            quiet = nxt >= len(order) or requests[order[nxt]][3] > tick + 1
            rep = rt.execute_next_tick(run_ahead=(mode == "always") or quiet)
        if rep is None:
            if nxt < len(order):
                tick = requests[order[nxt]][3]
                continue
            break
        log.append(rep)
        snaps.append((rt.pool_free_count(), [tuple(rt.sequence_blocks(s)) for s in ids if s is not None]))
        tick += 1
        assert len(log) < 10000
    return ids, log, snaps


def assert_same(a, b):
    aid, alog, asnap = a
    bid, blog, bsnap = b
    assert aid == bid and len(alog) == len(blog)
    for t, ((ak, au), (bk, bu)) in enumerate(zip(alog, blog)):
        assert ak == bk, t
        assert len(au) == len(bu), t
        for x, y in zip(au, bu):
            for key in ("sequence_id", "batch_kind", "reused", "appended", "phase", "finish_reason",
                        "token", "released"):
                assert x[key] == y[key], (t, key, x, y)
            if x["token"] is not None:
                assert np.float32(x["probability"]) == np.float32(y["probability"]), (t, x, y)
        assert asnap[t] == bsnap[t], t


def arrivals(cfg, seed, n, prompt_range, new_range, spread):
    rng = np.random.default_rng(seed)
    reqs = []
    for i in range(n):
        plen = int(rng.integers(*prompt_range))
        reqs.append((rng.integers(0, cfg["vocab"], plen).astype(np.uint32), int(rng.integers(*new_range)), None,
                     int(rng.integers(0, spread)) if i else 0))
    return reqs


def with_stops(serial_rt, requests, picks):
    """Stop tokens that a run without them generates mid-sequence, for the requests in picks."""
    ids, _, _ = drive(serial_rt, requests, None)
    out = list(requests)
    for i in picks:
        gen = serial_rt.generated(ids[i])
        if len(gen) > 6:
            p, n, _, arr = out[i]
            out[i] = (p, n, int(gen[len(gen) // 2]), arr)
    return out


@pytest.mark.parametrize("graph", [True, False])
def test_run_ahead_matches_serial_with_arrivals_and_stops(graph):
    """C1's tiny Llama, 12 requests arriving over 40 ticks, three of them with stop tokens
    that occur mid-run; the flag on every call (submits drop enqueued ticks) and only on quiet
    calls (nothing is dropped)."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    print(f"run ahead: C1 arrivals, graph={graph}", flush=True)
    cfg = TINY_LLAMA_C1
    weights = random_weights(cfg, seed=5)
    kw = dict(max_batch=8)
    reqs = arrivals(cfg, 21, 12, (10, 90), (12, 48), 40)
    reqs = with_stops(make_runtime(cfg, weights, graph, kw), reqs, (1, 4, 7))
    assert sum(r[2] is not None for r in reqs) >= 2
    base = drive(make_runtime(cfg, weights, graph, kw), reqs, None)
    assert any(u["finish_reason"] == 0 for _, us in base[1] for u in us)  # a stop-token finish
    for mode in ("always", "quiet"):
        rt = make_runtime(cfg, weights, graph, kw)
        assert_same(base, drive(rt, reqs, mode))
        c = rt.run_ahead_counters()
        print(f"{mode}: {c}", flush=True)
        assert c["kept"] > 20
        if mode == "always":
            assert c["dropped"] > 0
        else:
            assert c["dropped"] == 0
        assert rt.pool_free_count() == 4096


@pytest.mark.parametrize("weight_dtype,kv_dtype", [("f32", "f32"), ("f32", "bf16"), ("bf16", "f32")])
def test_run_ahead_more_decoding_sequences_than_the_batch(weight_dtype, kv_dtype):
    """12 sequences decoding at once with max_batch 4: a tick's rows come partly from the
    previous tick (fed on the device) and partly from sequences that sat out (ids from the
    host).  Also over a bf16 KV pool and bf16-stored weights."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    print(f"run ahead: batch-limited decode, weights {weight_dtype}, KV {kv_dtype}", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=6)
    kw = dict(max_batch=4)
    reqs = arrivals(cfg, 22, 12, (5, 40), (20, 40), 1)
    mk = lambda: make_runtime(cfg, weights, True, kw, weight_dtype=weight_dtype, kv_dtype=kv_dtype)
    base = drive(mk(), reqs, None)
    rt = mk()
    assert_same(base, drive(rt, reqs, "quiet"))
    c = rt.run_ahead_counters()
    print(f"counters {c}", flush=True)
    assert c["kept"] > 30 and c["dropped"] == 0


def test_run_ahead_at_the_sequence_length_limit():
    """max_seq 80 with prompts of 60-78 tokens: sequences finish by length, some on a tick
    that has no row for them, while the others keep decoding across block boundaries."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    print("run ahead: sequence-length limit", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=7)
    kw = dict(max_batch=8, max_seq=80)
    reqs = arrivals(cfg, 23, 6, (60, 79), (30, 40), 3)
    base = drive(make_runtime(cfg, weights, True, kw), reqs, None)
    assert any(u["finish_reason"] == 3 for _, us in base[1] for u in us)  # SequenceLength
    rt = make_runtime(cfg, weights, True, kw)
    assert_same(base, drive(rt, reqs, "always"))
    assert rt.run_ahead_counters()["kept"] > 5


@pytest.mark.parametrize("sampler,graph", [((0.8, 20, 0.9, 42), True), ((0.8, 20, 0.9, 42), False),
                                           ((0.9, 3000, 0.95, 7), True)])
def test_run_ahead_sampled_matches_serial(sampler, graph):
    """A sampled session run ahead: each tick's sampler states continue on the device from the
    previous tick's draws (rows fed from it) or come from the host (rows that sat out).  Tokens,
    probabilities, finish reasons and pool state equal serial calls', with submits between ticks
    and more decoding sequences than the batch; top-k 3000 samples from the reserved area."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    print(f"run ahead: sampled {sampler}, graph={graph}", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=3, std=0.05)
    kw = dict(max_batch=6)
    reqs = arrivals(cfg, 24, 10, (8, 60), (16, 40), 12)
    base = drive(make_runtime(cfg, weights, graph, kw, sampler=sampler), reqs, None)
    rt = make_runtime(cfg, weights, graph, kw, sampler=sampler)
    assert_same(base, drive(rt, reqs, "always"))
    c = rt.run_ahead_counters()
    print(f"counters {c}", flush=True)
    assert c["kept"] > 20 and c["dropped"] > 0


class _Ahead:
    """A Runtime whose every tick asks to run ahead, for the oracle comparison's driver."""

    def __init__(self, rt):
        self.rt = rt

    def execute_next_tick(self):
        return self.rt.execute_next_tick(run_ahead=True)

    def __getattr__(self, name):
        return getattr(self.rt, name)


def test_run_ahead_matches_reference(orc):
    """C1 through the oracle comparison of tests/test_gpu_model.py, every tick run ahead:
    packing, reports, released blocks and tokens as the reference scheduler's."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    print("run ahead: C1 against the oracle", flush=True)
    cfg = TINY_LLAMA_C1
    weights = random_weights(cfg, seed=0)
    model, ref = oracle_scheduler(orc, cfg, weights, {})
    rt = make_runtime(cfg, weights, True, {})
    _, ties = compare(model, ref, _Ahead(rt), c1_requests(0))
    assert ties == 0
    assert rt.run_ahead_counters()["kept"] > 20


def test_run_ahead_c4_shape_batch_64():
    """The C4 model shape at decode batch 64 (64 requests, 32-token prompts, 12 new tokens):
    ticks run ahead equal serial ones."""
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, random_weights

    print("run ahead: C4 shape batch 64", flush=True)
    cfg = QWEN2_05B_C4
    weights = random_weights(cfg, seed=0, qkv_bias=True)
    rng = np.random.default_rng(65)
    reqs = [(rng.integers(0, cfg["vocab"], 32).astype(np.uint32), 12, None, 0) for _ in range(64)]
    kw = dict(max_batch=64, max_seq=64)
    base = drive(make_runtime(cfg, weights, True, kw, num_blocks=512), reqs, None)
    rt = make_runtime(cfg, weights, True, kw, num_blocks=512)
    del weights
    assert_same(base, drive(rt, reqs, "quiet"))
    c = rt.run_ahead_counters()
    print(f"counters {c}", flush=True)
    assert c["kept"] >= 10 and c["dropped"] == 0


def test_observers_before_submit_leave_weights_open():
    """The counters, the tick profile, the last batch and the last logits report an empty state
    before the first submit and create no scheduler: the weights can still be set."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    cfg = dict(TINY_LLAMA_C1, layers=1)
    from ferrisinfer_amd.runtime import Runtime

    rt = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                 cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"], tie=cfg["tie"], graph_decode=True)
    assert rt.run_ahead_counters() == dict(launched=0, kept=0, dropped=0, last_ahead=False)
    assert rt.graph_counters() == dict(replays=0, captures=0, drops=0)
    assert rt.last_tick_profile()["total"] == 0.0
    assert rt.last_logits().shape[0] == 0
    rt.set_weights(random_weights(cfg, seed=1))  # not frozen by the observers above
    seq = rt.submit(np.arange(5, dtype=np.uint32), max_new_tokens=3)
    while rt.execute_next_tick(run_ahead=True) is not None:
        pass
    assert len(rt.generated(seq)) == 3
