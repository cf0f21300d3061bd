"""End-to-end parity of the GPU runtime (batched ticks over the HIP backend) with the CPU
oracle's restatement of the reference scheduler + sessions (sequential per-sequence
forwards).  Tick compositions, reports and block accounting must be identical; each tick's
packed metadata (positions, slot mapping, cu_seqlens, context lengths, block tables,
copy-on-write list) must equal the oracle packer's bit for bit; greedy tokens must be
identical except where the oracle's own top-2 logit gap is a near tie (< 1e-4 relative),
where summation order may legitimately pick the other token."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def build_pair(orc, cfg, weights, sched_kw, num_blocks=4096, kv_dtype="f32", sampler=None):
    from ferrisinfer_amd.runtime import Runtime

    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                      cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                      tie=cfg["tie"])
    model.set_weights(weights)
    ref = orc.Scheduler(model, page_size=16, sampler=sampler, **sched_kw)
    ref.attach_packer(num_blocks, 16)
    gpu = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                  cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                  tie=cfg["tie"], num_blocks=num_blocks, block_size=16, kv_dtype=kv_dtype,
                  sampler=sampler, **sched_kw)
    gpu.set_weights(weights)
    return model, ref, gpu


PACK_KEYS = ("positions", "slot_mapping", "cu_seqlens", "context_lens", "block_tables",
             "copy_src", "copy_dst", "copy_count", "sequence_ids")


def drive(sched, requests, packs=None, after_tick=None):
    ids = [sched.submit(p, max_new_tokens=n) for p, n in requests]
    ticks = []
    while True:
        t = sched.execute_next_tick()
        if t is None:
            break
        ticks.append(t)
        if packs is not None:
            packs.append(sched.packed() if hasattr(sched, "packed") else sched.last_batch())
        if after_tick is not None:
            after_tick(ids)
        assert len(ticks) < 10000
    return ids, ticks


def oracle_pages_are_logical(ref, requests):
    """After-tick hook for the oracle scheduler: every live sequence's own paged storage holds
    logical block i in page i (a fresh or imported per-sequence storage hands pages out of its
    LIFO list [n-1 .. 0] in logical order, runtime/paged_kv.rs:329-389, 469-527, 794-796), so the
    block ids of the oracle's released lists are logical block indices."""
    def check(ids):
        for seq, (prompt, _) in zip(ids, requests):
            tokens = min(orc_cached_tokens(ref, seq), len(prompt))
            if tokens == 0:
                continue
            pages = ref.session_blocks(seq, 0, tokens)
            if pages is not None:
                assert pages == list(range(len(pages))), (seq, pages)
    return check


def orc_cached_tokens(ref, seq):
    from oracle import scheduler_sequence_state

    return scheduler_sequence_state(ref, seq)["cached_tokens"]


def gpu_released_as_logical(gticks, gpacks, block_size=16):
    """The GPU runtime's released (owner, layer, pool block id) entries mapped to (owner, layer,
    logical block index) through the owner's block table as packed up to that tick."""
    tables, out = {}, []
    for (_, updates), pack in zip(gticks, gpacks):
        for i, seq in enumerate(pack["sequence_ids"]):
            n = (int(pack["context_lens"][i]) + block_size - 1) // block_size
            tables[int(seq)] = [int(b) for b in pack["block_tables"][i][:n]]
        tick = []
        for u in updates:
            tick.append([(o, l, tables[o].index(b)) for o, l, b in u["released"]])
        out.append(tick)
    return out


def near_tie(model, history, vocab):
    logits = model.forward_logits(np.asarray(history, np.uint32))[-1]
    top = np.sort(logits)[-2:]
    return float(top[1] - top[0]) <= 1e-4 * max(1.0, abs(float(top[1])))


def compare(model, ref, gpu, requests):
    rpacks, gpacks = [], []
    rid, rticks = drive(ref, requests, rpacks, after_tick=oracle_pages_are_logical(ref, requests))
    gid, gticks = drive(gpu, requests, gpacks)
    assert rid == gid
    assert len(rticks) == len(gticks)
    for i, (a, b) in enumerate(zip(rpacks, gpacks)):
        assert a["kind"] == b["kind"], i
        for key in PACK_KEYS:
            assert np.array_equal(a[key], b[key]), (i, key, a[key], b[key])
    g_released = gpu_released_as_logical(gticks, gpacks)
    for t, ((rk, ru), (gk, gu)) in enumerate(zip(rticks, gticks)):
        assert rk == gk
        assert [u["sequence_id"] for u in ru] == [u["sequence_id"] for u in gu]
        for j, (a, b) in enumerate(zip(ru, gu)):
            for key in ("batch_kind", "reused", "appended", "phase", "finish_reason"):
                assert a[key] == b[key], (key, a, b)
            # released prefix blocks: same owners, layers, logical blocks and order
            assert a["released"] == g_released[t][j], (t, a["released"], g_released[t][j])
            assert (a["token"] is None) == (b["token"] is None)
    ties = 0
    for seq, (prompt, _) in zip(rid, requests):
        r = ref.generated(seq)
        g = gpu.generated(seq)
        assert len(r) == len(g)
        for i, (a, b) in enumerate(zip(r, g)):
            if a != b:
                hist = list(prompt) + r[:i]
                assert near_tie(model, hist, None), f"seq {seq} token {i}: {a} vs {b}"
                ties += 1
                break
    return rticks, ties


def test_c1_tiny_llama_greedy_matches_reference(orc):
    """tiny Llama (4 layers, H 256, 8/2 heads, D 32, F 688, V 4096),
    4 requests (16/24/32/48-token prompts), 32 greedy tokens each, block 16, continuous
    batching with the reference scheduler defaults."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    cfg = TINY_LLAMA_C1
    weights = random_weights(cfg, seed=0)
    model, ref, gpu = build_pair(orc, cfg, weights, {})
    ticks, ties = compare(model, ref, gpu, c1_requests(0))
    assert ties == 0
    assert gpu.pool_free_count() == 4096  # every block returned once all requests finished


def test_bf16_kv_pool_runtime_tracks_reference(orc):
    """The runtime over a bf16 KV pool (rows narrowed to bf16 with nearest even on append,
    widened on read): the scheduler's ticks, reports and packing metadata are value-independent
    and must equal the oracle's exactly; greedy tokens must equal the f32 reference's except
    where its top-2 logit gap is within the bf16 storage error (2e-2 relative), after which
    that sequence is not compared further."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=11)
    model, ref, gpu = build_pair(orc, cfg, weights, {}, kv_dtype="bf16")
    requests = c1_requests(2)
    rpacks, gpacks = [], []
    rid, rticks = drive(ref, requests, rpacks)
    gid, gticks = drive(gpu, requests, gpacks)
    assert rid == gid and len(rticks) == len(gticks)
    for i, (a, b) in enumerate(zip(rpacks, gpacks)):
        for key in PACK_KEYS:
            assert np.array_equal(a[key], b[key]), (i, key)
    matched = 0
    for seq, (prompt, _) in zip(rid, requests):
        r, g = ref.generated(seq), gpu.generated(seq)
        assert len(r) == len(g)
        for i, (a, b) in enumerate(zip(r, g)):
            if a != b:
                logits = model.forward_logits(np.asarray(list(prompt) + r[:i], np.uint32))[-1]
                top = np.sort(logits)[-2:]
                assert float(top[1] - top[0]) <= 2e-2 * max(1.0, abs(float(top[1]))), (seq, i, a, b)
                break
            matched += 1
    assert matched >= len(requests) * 8  # most tokens agree before any near tie
    assert gpu.pool_free_count() == 4096


def test_prefix_sharing_and_chunking_match_reference(orc):
    """Shared prompt prefixes (min_share 16, block-aligned and not), chunked prefill (chunk 20,
    batch budget 50), decode fairness with batch size 3: same ticks, reuse counts, released
    blocks and tokens as the reference scheduler."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=3)
    rng = np.random.default_rng(7)
    base = rng.integers(0, cfg["vocab"], size=40).astype(np.uint32)
    reqs = [
        (base.copy(), 6),                                                       # source
        (np.concatenate([base[:37], rng.integers(0, 4096, 9)]).astype(np.uint32), 5),  # shares 37
        (np.concatenate([base[:32], rng.integers(0, 4096, 3)]).astype(np.uint32), 4),  # shares 32
        (base.copy(), 3),                                                       # whole prompt
        (rng.integers(0, 4096, 23).astype(np.uint32), 7),                       # unrelated
    ]
    kw = dict(max_batch=3, max_chunk=20, max_batch_tokens=50, min_share=16)
    model, ref, gpu = build_pair(orc, cfg, weights, kw)
    ticks, ties = compare(model, ref, gpu, reqs)
    assert any(u["reused"] > 0 for _, us in ticks for u in us)
    assert gpu.pool_free_count() == 4096


SAMPLERS = [(0.8, 20, 0.9, 42), (1.3, 50, 1.0, 0)]


@pytest.mark.parametrize("sampler", [(0.9, 3000, 1.0, 7), (1.0, 4096, 1.0, 5)])
def test_sampled_large_top_k_ticks_track_reference(orc, sampler):
    """Top-k above 1024 through the runtime (which reserves the sampler's area), up to the whole
    4096-token vocabulary, on the C1 requests.  Ticks and reports equal the oracle scheduler's.
    Every sampled token equals the reference's sample_last_token on the logits row the runtime
    sampled from (fr_last_logits), with the sequence's state (the seed's, advanced once per
    earlier token: no prefix imports here): exact, the sampler's own contract.  Those logits
    equal the reference's forward to 1e-4 (checked on every sequence's first row).  Tokens are
    not compared with the oracle scheduler's: with thousands of nearly flat weights, logits that
    differ in their last bits move a draw that falls near a partial sum to the neighbouring
    candidate, and every later token of that sequence with it."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    print(f"sampled ticks, large top-k {sampler}", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=3, std=0.05)
    requests = c1_requests(0)
    model, ref, gpu = build_pair(orc, cfg, weights, {}, sampler=sampler)
    rid, rticks = drive(ref, requests)
    rows = []  # per GPU tick: {sequence id: logits row}
    gid, gticks = drive(gpu, requests, after_tick=lambda _: rows.append(
        dict(zip((int(s) for s in gpu.last_batch()["sequence_ids"]), gpu.last_logits()))))
    assert rid == gid and len(rticks) == len(gticks)
    for (rk, ru), (gk, gu) in zip(rticks, gticks):
        assert rk == gk
        for a, b in zip(ru, gu):
            for key in ("sequence_id", "reused", "appended", "phase", "finish_reason"):
                assert a[key] == b[key], (key, a, b)
    # a sequence's i-th generated token is drawn from the i-th tick that sampled it (prompts
    # prefill in one tick here; a tick reports the token it appends, drawn the tick before)
    temperature, top_k, top_p, seed = sampler
    drawn = 0
    for seq, (prompt, _) in zip(gid, requests):
        seq_rows = [r[seq] for r in rows if seq in r]
        generated = gpu.generated(seq)
        assert len(seq_rows) >= len(generated)
        want = model.forward_logits(np.asarray(prompt, np.uint32))[-1]  # the first draw's row
        np.testing.assert_allclose(seq_rows[0], want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
        state = orc.sampler_state_new(seed)
        for i, tok in enumerate(generated):
            token, _, state = orc.sample_last_token(seq_rows[i], temperature, top_k, top_p, state)
            assert tok == token, (seq, i, tok, token)
            drawn += 1
    print(f"large top-k {sampler}: {drawn} draws equal the reference sampler's on the runtime's logits", flush=True)
    assert drawn == sum(n for _, n in requests)
    assert gpu.pool_free_count() == 4096


@pytest.mark.parametrize("sampler", SAMPLERS)
def test_sampled_ticks_match_reference(orc, sampler):
    """A sampling SessionConfig (runtime/sampler.rs:121-241 per sequence, xorshift64* state
    per session): the C1 requests and the prefix-sharing set under the same scheduler limits
    as above.  Every sequence's tokens must equal the reference's exactly: the draws consume
    the per-sequence states in the reference's order, including a whole-history import from a
    source that drew earlier in the same tick."""
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    print(f"sampled ticks sampler={sampler}", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = random_weights(cfg, seed=3, std=0.05)
    rng = np.random.default_rng(7)
    base = rng.integers(0, cfg["vocab"], size=40).astype(np.uint32)
    sharing = [
        (base.copy(), 6),
        (np.concatenate([base[:37], rng.integers(0, 4096, 9)]).astype(np.uint32), 5),
        (base.copy(), 3),
        (rng.integers(0, 4096, 23).astype(np.uint32), 7),
    ]
    cases = [(c1_requests(0), {}),
             (sharing, dict(max_batch=3, max_chunk=20, max_batch_tokens=50, min_share=16))]
    for requests, kw in cases:
        model, ref, gpu = build_pair(orc, cfg, weights, kw, sampler=sampler)
        rid, rticks = drive(ref, requests)
        gid, gticks = drive(gpu, requests)
        assert rid == gid and len(rticks) == len(gticks)
        for (rk, ru), (gk, gu) in zip(rticks, gticks):
            assert rk == gk
            for a, b in zip(ru, gu):
                for key in ("sequence_id", "reused", "appended", "phase", "finish_reason", "token"):
                    assert a[key] == b[key], (key, a, b)
                if a["token"] is not None:
                    assert abs(a["probability"] - b["probability"]) <= 1e-4 * a["probability"]
        for seq in rid:
            assert ref.generated(seq) == gpu.generated(seq), seq
        assert gpu.pool_free_count() == 4096


def test_sampler_config_limits(orc):
    from ferrisinfer_amd.runtime import Runtime
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1

    cfg = TINY_LLAMA_C1
    Runtime(cfg["hidden"], cfg["intermediate"], 1, cfg["heads"], cfg["kv_heads"], cfg["vocab"],
            sampler=(0.8, 2000, 0.9, 0)).close()  # above 1024: served from a reserved area
    Runtime(cfg["hidden"], cfg["intermediate"], 1, cfg["heads"], cfg["kv_heads"], 1000,
            sampler=(0.8, 2000, 0.9, 0)).close()  # clamps to the 1000-token vocabulary
    Runtime(cfg["hidden"], cfg["intermediate"], 1, cfg["heads"], cfg["kv_heads"], cfg["vocab"],
            sampler=(0.0, 2000, 0.9, 0)).close()  # greedy: top_k unused


def test_runtime_errors(orc):
    from ferrisinfer_amd import FerrisError
    from ferrisinfer_amd.runtime import Runtime
    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, random_weights

    cfg = dict(TINY_LLAMA_C1, layers=1)
    rt = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                 cfg["vocab"], num_blocks=4, block_size=16, max_seq=256)
    w = random_weights(cfg)
    del w["norm.weight"]
    rt.set_weights(w)
    with pytest.raises(FerrisError) as e:
        rt.submit([1, 2, 3])
    assert e.value.kind == "MissingWeight"
    rt2 = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                  cfg["vocab"], num_blocks=2, block_size=16, max_seq=256)
    rt2.set_weights(random_weights(cfg))
    with pytest.raises(FerrisError) as e:
        rt2.submit([4096])
    assert e.value.kind == "InvalidShape"  # token id out of vocabulary (attention.rs:35-40)
    rt2.submit(list(range(40)), max_new_tokens=1)
    with pytest.raises(FerrisError) as e:
        rt2.execute_next_tick()  # 40 tokens need 3 blocks, the pool has 2
    assert e.value.kind == "Runtime"


def test_c4_qwen2_shape_matches_reference(orc):
    """BASELINE config C4's model (Qwen2-0.5B shape: 24 layers, H 896, 14/2 heads, D 64,
    F 4864, V 151936, tied embeddings, q/k/v biases, theta 1e6; f32 N(0, 0.02) weights) under
    the continuous-batching driver with Poisson arrival ticks, on a declared subset of the C4
    workload that the CPU oracle finishes in seconds: its first 3 requests with prompts cut to
    64 tokens and 4 new tokens each.  Tick log and greedy tokens must match the reference."""
    from ferrisinfer_amd.runtime import Runtime
    from ferrisinfer_amd.workloads import (QWEN2_05B_C4, c4_requests, random_weights,
                                           run_continuous)

    cfg = QWEN2_05B_C4
    weights = random_weights(cfg, seed=0, qkv_bias=True)
    reqs = c4_requests(seed=0)[:3]
    for r in reqs:
        r["prompt"] = r["prompt"][:64]
        r["max_new_tokens"] = 4
    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                      cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                      tie=cfg["tie"])
    model.set_weights(weights)
    ref = orc.Scheduler(model, max_batch=64)
    rrep = run_continuous(ref, reqs)
    gpu = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                  cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                  tie=True, max_batch=64, num_blocks=256, block_size=16)
    gpu.set_weights(weights)
    del weights
    grep = run_continuous(gpu, reqs)
    strip = [{k: t[k] for k in ("tick", "kind", "batch", "generated", "appended")}
             for t in rrep["ticks"]]
    assert strip == [{k: t[k] for k in ("tick", "kind", "batch", "generated", "appended")}
                     for t in grep["ticks"]]
    for seq, r in zip(rrep["sequence_ids"], reqs):
        a, b = ref.generated(seq), gpu.generated(seq)
        assert len(a) == len(b) == 4
        for i, (x, y) in enumerate(zip(a, b)):
            if x != y:
                assert near_tie(model, list(r["prompt"]) + a[:i], None), (seq, i, x, y)
                break


def test_c4_qwen2_shape_reaches_decode_batch_64(orc):
    """BASELINE config C4's model (Qwen2-0.5B shape, 24 layers, tied, q/k/v biases) at the
    headline decode batch: 64 requests of 32-token prompts and 8 new tokens under max_batch 64,
    so the decode ticks carry all 64 sequences.  Ticks, reports, released blocks and every
    tick's packing must equal the oracle's; greedy tokens too, except at a reported near tie."""
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, random_weights

    print("C4 shape at decode batch 64", flush=True)
    cfg = QWEN2_05B_C4
    weights = random_weights(cfg, seed=0, qkv_bias=True)
    rng = np.random.default_rng(64)
    requests = [(rng.integers(0, cfg["vocab"], 32).astype(np.uint32), 8) for _ in range(64)]
    model, ref, gpu = build_pair(orc, cfg, weights, dict(max_batch=64, max_seq=64), num_blocks=512)
    del weights
    ticks, ties = compare(model, ref, gpu, requests)
    assert sum(1 for kind, us in ticks if kind == 1 and len(us) == 64) >= 7
    print(f"C4 batch 64: {len(ticks)} ticks, near ties {ties}", flush=True)
    assert gpu.pool_free_count() == 512


def test_c4_width_long_prompts_match_reference(orc):
    """BASELINE config C4's prompt range at the C4 width (H 896, 14/2 heads, D 64, F 4864, full
    vocab 151936, tied embeddings, q/k/v biases, theta 1e6; 4 of its 24 layers so the oracle
    finishes in seconds): 3 requests with 700-, 1500- and 2048-token prompts (the lognormal
    workload's clip) under the bench's scheduler settings (max batch 64, max_seq 4096, default
    256-token chunks and 1024-token tick budget), so prefill runs as multi-chunk cached-prefix
    ticks at the f32-pool prefill kernel's GQA-7 shape.  Ticks, reports, released blocks and
    every tick's packing equal the oracle's; greedy tokens too, except at a near tie."""
    from ferrisinfer_amd import seeded
    from ferrisinfer_amd.seeded import tag_of
    from ferrisinfer_amd.workloads import QWEN2_05B_C4, random_weights

    print("C4 width, 700/1500/2048-token prompts", flush=True)
    cfg = dict(QWEN2_05B_C4, layers=4)
    weights = random_weights(cfg, seed=3, qkv_bias=True)
    requests = [(seeded.integers(3, tag_of(f"c4r.prompt.{i}"), n, 0, cfg["vocab"] - 1).astype(np.uint32), 6)
                for i, n in enumerate((700, 1500, 2048))]
    model, ref, gpu = build_pair(orc, cfg, weights, dict(max_batch=64, max_seq=4096, max_gen=512),
                                 num_blocks=1024)
    del weights
    ticks, ties = compare(model, ref, gpu, requests)
    prefill_ticks = sum(1 for kind, _ in ticks if kind == 0)
    assert prefill_ticks >= (700 + 1500 + 2048) // 1024  # chunked over several ticks
    print(f"C4 long prompts: {len(ticks)} ticks ({prefill_ticks} prefill), near ties {ties}", flush=True)
    assert gpu.pool_free_count() == 1024


def test_c5_width_bf16_runtime_tracks_reference(orc):
    """BASELINE config C5's layer shape through fr_execute_next_tick: 2 of its 32 layers
    (H 4096, 32/8 heads, D 128, FFN 14336, theta 5e5), the full 128256-token vocabulary with an
    untied head, bf16-stored weights (weight_dtype "bf16") and a bf16 KV pool, under the C5
    step's 2048-token tick budget with 256-token chunks (a 700-token prompt prefills in three
    cached-prefix ticks).  Against the oracle scheduler on the same bf16-valued weights in f32
    (what the reference's loader hands its kernels, io/safetensors.rs:540-542): ticks, reports
    and every tick's packing are exact; greedy tokens equal the reference's except where its
    top-2 logit gap is within the bf16 rounding of activations and KV (2e-2 relative), after
    which that sequence is not compared further.  Weights and prompts are drawn from
    ferrisinfer_amd.seeded."""
    from ferrisinfer_amd import seeded
    from ferrisinfer_amd.bf16_decoder import LLAMA3_8B_C5
    from ferrisinfer_amd.seeded import tag_of
    from ferrisinfer_amd.workloads import random_weights

    print("C5 width: drawing 1.49e9 seeded weights", flush=True)
    cfg = dict(LLAMA3_8B_C5, layers=2)
    weights = bf16_rounded(orc, random_weights(cfg, seed=5))
    requests = [(seeded.integers(5, tag_of(f"c5r.prompt.{i}"), n, 0, cfg["vocab"] - 1).astype(np.uint32), 4)
                for i, n in enumerate((96, 288, 700))]
    kw = dict(max_batch=256, max_seq=10240, max_gen=512, max_chunk=256, max_batch_tokens=2048)
    print("C5 width: oracle model and GPU runtime", flush=True)
    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                      cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"], tie=cfg["tie"])
    model.set_weights(weights)
    ref = orc.Scheduler(model, page_size=16, **kw)
    ref.attach_packer(1024, 16)
    from ferrisinfer_amd.runtime import Runtime

    gpu = Runtime(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                  cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"], tie=cfg["tie"], num_blocks=1024,
                  block_size=16, kv_dtype="bf16", weight_dtype="bf16", **kw)
    gpu.set_weights(weights)
    del weights
    rpacks, gpacks = [], []
    gid, gticks = drive(gpu, requests, gpacks)
    print(f"C5 width: GPU runtime done in {len(gticks)} ticks; oracle scheduler next", flush=True)
    rid, rticks = drive(ref, requests, rpacks)
    assert rid == gid and len(rticks) == len(gticks)
    for i, (a, b) in enumerate(zip(rpacks, gpacks)):
        assert a["kind"] == b["kind"], i
        for key in PACK_KEYS:
            assert np.array_equal(a[key], b[key]), (i, key)
    for (rk, ru), (gk, gu) in zip(rticks, gticks):
        assert rk == gk
        for a, b in zip(ru, gu):
            for key in ("sequence_id", "reused", "appended", "phase", "finish_reason"):
                assert a[key] == b[key], (key, a, b)
    assert sum(1 for kind, _ in gticks if kind == 0) >= 3  # the 700-token prompt's chunks
    matched = 0
    for seq, (prompt, _) in zip(rid, requests):
        r, g = ref.generated(seq), gpu.generated(seq)
        assert len(r) == len(g)
        for i, (a, b) in enumerate(zip(r, g)):
            if a != b:
                logits = model.forward_logits(np.asarray(list(prompt) + r[:i], np.uint32))[-1]
                top = np.sort(logits)[-2:]
                assert float(top[1] - top[0]) <= 2e-2 * max(1.0, abs(float(top[1]))), (seq, i, a, b)
                break
            matched += 1
    print(f"C5 width: {matched} of {sum(n for _, n in requests)} tokens matched before any near tie", flush=True)
    assert matched >= 2 * len(requests)
    assert gpu.pool_free_count() == 1024
    gpu.close()


def bf16_rounded(orc, weights):
    """The weights a bf16 checkpoint holds: every matrix rounded to bf16 (nearest even) and
    widened back, which is what the reference's loader hands its f32 kernels
    (io/safetensors.rs:540-542); vectors (norms, biases) stay f32."""
    return {k: (orc.bf16_to_f32(orc.f32_to_bf16(v)) if np.ndim(v) == 2 else v) for k, v in weights.items()}


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_bf16_weight_runtime_tracks_reference(orc, kv_dtype):
    """The runtime serving bf16-stored projection weights and head (weight_dtype "bf16",
    fi_gemm_bf16 / fi_gemm_bf16_swiglu / fi_lm_head_argmax_bf16), over an f32 or bf16 KV pool,
    against the oracle scheduler on the same bf16-valued weights in f32.  Ticks, reports and
    every tick's packing are exact; greedy tokens equal the reference's except where its top-2
    logit gap is within the bf16 activation rounding (2e-2 relative), after which that sequence
    is not compared further.  The graph-replayed runtime on the same weights equals the eager
    one bit for bit."""
    from test_gpu_graph import assert_same_run, make_runtime

    from ferrisinfer_amd.workloads import TINY_LLAMA_C1, c1_requests, random_weights

    print(f"bf16 weights runtime kv={kv_dtype}", flush=True)
    cfg = dict(TINY_LLAMA_C1, layers=2)
    weights = bf16_rounded(orc, random_weights(cfg, seed=21))
    model = orc.Model(cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"],
                      cfg["kv_heads"], cfg["vocab"], cfg["max_pos"], cfg["eps"], cfg["theta"],
                      tie=cfg["tie"])
    model.set_weights(weights)
    ref = orc.Scheduler(model, page_size=16)
    ref.attach_packer(4096, 16)
    gpu = make_runtime(cfg, weights, False, {}, weight_dtype="bf16", kv_dtype=kv_dtype)
    requests = c1_requests(5)
    rpacks, gpacks = [], []
    rid, rticks = drive(ref, requests, rpacks)
    gid, gticks = drive(gpu, requests, gpacks)
    assert rid == gid and len(rticks) == len(gticks)
    for i, (a, b) in enumerate(zip(rpacks, gpacks)):
        for key in PACK_KEYS:
            assert np.array_equal(a[key], b[key]), (i, key)
    for (rk, ru), (gk, gu) in zip(rticks, gticks):
        assert rk == gk
        for a, b in zip(ru, gu):
            for key in ("sequence_id", "reused", "appended", "phase", "finish_reason"):
                assert a[key] == b[key], (key, a, b)
    matched = 0
    for seq, (prompt, _) in zip(rid, requests):
        r, g = ref.generated(seq), gpu.generated(seq)
        assert len(r) == len(g)
        for i, (a, b) in enumerate(zip(r, g)):
            if a != b:
                logits = model.forward_logits(np.asarray(list(prompt) + r[:i], np.uint32))[-1]
                top = np.sort(logits)[-2:]
                assert float(top[1] - top[0]) <= 2e-2 * max(1.0, abs(float(top[1]))), (seq, i, a, b)
                break
            matched += 1
    print(f"bf16 weights: {matched} tokens matched before any near tie", flush=True)
    assert matched >= len(requests) * 8
    assert gpu.pool_free_count() == 4096
    eager = make_runtime(cfg, weights, False, {}, weight_dtype="bf16", kv_dtype=kv_dtype)
    graph = make_runtime(cfg, weights, True, {}, weight_dtype="bf16", kv_dtype=kv_dtype)
    assert_same_run(eager, graph, requests)
