"""The oracle's sampled sessions (runtime/session.rs:104-139, 188-212, 349-406): a non-greedy
SamplerConfig takes the last row's logits through sample_last_token with the session's
xorshift64* state (one draw per processed chunk or token); a greedy one keeps the fused argmax
head and never draws; importing a prefix restarts the state from the seed, or takes the
source's state when the whole source history is imported.  These pin the session semantics
the GPU runtime's sampled ticks are compared against."""
import numpy as np

from ferrisinfer_amd.workloads import random_weights

CFG = dict(hidden=32, intermediate=48, layers=2, heads=4, kv_heads=2, vocab=97, max_pos=256,
           eps=1e-5, theta=10000.0, tie=False)
SAMPLED = (0.8, 5, 0.9, 7)


def model(orc):
    m = orc.Model(CFG["hidden"], CFG["intermediate"], CFG["layers"], CFG["heads"],
                  CFG["kv_heads"], CFG["vocab"], CFG["max_pos"], CFG["eps"], CFG["theta"])
    # std 0.5 makes the logits spread enough for top-k / top-p to matter
    w = random_weights(CFG, seed=11, std=0.5)
    m.set_weights(w)
    return m, w["output.weight"]


def xorshift(state, n=1):
    for _ in range(n):
        state ^= state >> 12
        state ^= (state << 25) & 0xFFFFFFFFFFFFFFFF
        state ^= state >> 27
    return state


def test_sampled_session_draws_once_per_processed_chunk(orc):
    m, out = model(orc)
    s = orc.Session(m, max_seq=64, max_gen=64)
    s.set_sampler(*SAMPLED)
    start = orc.sampler_state_new(SAMPLED[3])
    assert s.sampler_state == start
    s.prefill(np.array([3, 14, 15, 92, 65], np.uint32))
    assert s.sampler_state == xorshift(start, 1)
    state = start
    for step in range(12):
        # the sample of the last processed position, recomputed from its hidden row
        tok, prob, state = orc.sample_last_token(
            orc.matmul_rhs_transposed(s.last_hidden()[None, :], out), *SAMPLED[:3], state)
        assert s.last_sample()[0] == tok
        assert abs(s.last_sample()[1] - prob) <= 1e-6 * prob
        assert s.step()[0] == tok
        assert s.sampler_state == xorshift(start, step + 2)


def test_greedy_session_never_draws(orc):
    m, _ = model(orc)
    s = orc.Session(m, max_seq=64, max_gen=64)
    s.set_sampler(0.8, 1, 0.9, 7)  # top_k 1 is greedy (sampler.rs:40-42)
    start = s.sampler_state
    s.prefill(np.array([1, 2, 3], np.uint32))
    for _ in range(4):
        s.step()
    assert s.sampler_state == start


def test_prefix_import_restarts_or_copies_the_sampler_state(orc):
    m, _ = model(orc)
    src = orc.Session(m, max_seq=64, max_gen=64, page_size=4)
    src.set_sampler(*SAMPLED)
    src.prefill(np.array([5, 6, 7, 8, 9, 10], np.uint32))
    src.step()
    src.step()
    assert src.sampler_state == xorshift(orc.sampler_state_new(SAMPLED[3]), 3)
    whole = orc.Session(m, max_seq=64, max_gen=64, page_size=4)
    whole.set_sampler(*SAMPLED)
    whole.copy_prefix_from(src, src.position)
    assert whole.sampler_state == src.sampler_state
    assert whole.last_sample() == src.last_sample()
    # it then continues the source's sequence of draws exactly
    assert [whole.step()[0] for _ in range(5)] == [src.step()[0] for _ in range(5)]
    part = orc.Session(m, max_seq=64, max_gen=64, page_size=4)
    part.set_sampler(*SAMPLED)
    part.copy_prefix_from(src, 4)
    assert part.sampler_state == orc.sampler_state_new(SAMPLED[3])


def test_sampled_scheduler_matches_independent_sessions(orc):
    """Without prefix sharing every scheduled sequence is an independent session with the
    same sampler: its generated tokens are those of a lone session fed the same prompt."""
    m, _ = model(orc)
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, CFG["vocab"], size=n).astype(np.uint32) for n in (5, 9, 13)]
    sched = orc.Scheduler(m, max_batch=4, min_share=1000, sampler=SAMPLED)
    ids = [sched.submit(p, max_new_tokens=8) for p in prompts]
    while sched.execute_next_tick() is not None:
        pass
    for seq, p in zip(ids, prompts):
        s = orc.Session(m, max_seq=4096, max_gen=512)
        s.set_sampler(*SAMPLED)
        s.prefill(p)
        want = [s.step()[0] for _ in range(8)]
        assert sched.generated(seq) == want
