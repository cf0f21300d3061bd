"""GPU parity of fi_sample_tokens (device-side sample_last_token / argmax_last_token,
runtime/sampler.rs:77-241) against the oracle's restatement: tokens and xorshift64* states
bit-exact, probabilities within 1e-5 relative (the device expf may differ from the host's in
the last bit), over consecutive calls that carry the states."""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NAN = float("nan")

# (temperature, top_k, top_p): greedy by each of the three rules, the reference's
# chat_default, wide and narrow top-k / top-p, top_k 0 (k = 1 on the sampling path), the
# device maximum k, and NaN temperature / top_p (temperature -> EPSILON, top_p keeps every
# candidate).
CONFIGS = [
    (0.0, 20, 0.9),
    (0.7, 1, 0.9),
    (0.7, 20, 0.0),
    (0.7, 20, 0.9),
    (1.3, 40, 1.0),
    (0.7, 2, 0.5),
    (1.0, 1024, 0.95),
    (1.0, 0, 0.9),
    (0.5, 200, 1.0),
    (2.0, 64, 0.99),
    (NAN, 20, 0.9),
    (1.0, 50, NAN),
    (0.9, 1000, 0.3),
]


def u64_to_i64(states):
    return np.asarray(states, dtype=np.uint64).view(np.int64)


def run_device(ctx, logits_t, configs, states):
    """One fi_sample_tokens call; returns (tokens, probs, new_states as python ints)."""
    import torch

    rows = logits_t.shape[0]
    temp = torch.tensor([c[0] for c in configs], dtype=torch.float32, device="cuda")
    topk = torch.tensor([c[1] for c in configs], dtype=torch.int32, device="cuda")
    topp = torch.tensor([c[2] for c in configs], dtype=torch.float32, device="cuda")
    st = torch.from_numpy(u64_to_i64(states).copy()).cuda()
    tok = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    prob = torch.zeros(rows, dtype=torch.float32, device="cuda")
    ctx.sample_tokens(logits_t, temp, topk, topp, st, tok, prob)
    torch.cuda.synchronize()
    new_states = [int(x) for x in st.cpu().numpy().view(np.uint64)]
    return tok.cpu().numpy(), prob.cpu().numpy(), new_states


def is_greedy(t, k, p):
    return t <= 0.0 or k == 1 or p <= 0.0


def check_rows(orc, logits, configs, states, tok, prob, new_states, label):
    """Tokens and states exact.  Sampled rows: the probability within 1e-5 relative (both sides
    sum the same weights in the same order; a weight may differ in its last bit, device expf
    against the host's).  Greedy rows: the reference sums all `vocab`
    exponentials one after another in f32, the device in a tree, so the device value is held to
    1e-5 of the exact (f64) 1 / sum exp(l - max) and the oracle's to the recursive-summation
    bound (vocab - 1) * 2^-24 of it."""
    for r, (t, k, p) in enumerate(configs):
        rt, rp, rs = orc.sample_last_token(logits[r], t, k, p, states[r])
        assert tok[r] == rt, f"{label} row {r} cfg {(t, k, p)}: token {tok[r]} != {rt}"
        assert new_states[r] == rs, f"{label} row {r}: rng state differs"
        if math.isnan(rp):
            assert math.isnan(prob[r]), f"{label} row {r}: prob {prob[r]} != NaN"
        elif is_greedy(t, k, p):
            row = logits[r].astype(np.float64)
            exact = 1.0 / np.exp(row - row[rt]).sum()
            assert abs(prob[r] - exact) <= 1e-5 * exact, f"{label} row {r}: prob {prob[r]} vs {exact}"
            assert abs(rp - exact) <= (len(row) - 1) * 2.0**-24 * exact
        else:
            assert abs(prob[r] - rp) <= 1e-5 * abs(rp) + 1e-30, f"{label} row {r}: prob {prob[r]} vs {rp}"


def padded_logits(logits, pad):
    """Device copy of logits [rows, vocab] with row stride vocab + pad (a strided view)."""
    import torch

    rows, vocab = logits.shape
    buf = torch.zeros((rows, vocab + pad), dtype=torch.float32, device="cuda")
    view = buf[:, :vocab]
    view.copy_(torch.from_numpy(logits))
    return view


@pytest.mark.parametrize("vocab,pad", [(37, 0), (1000, 0), (32000, 0), (32000, 5), (151936, 0), (151937, 3)])
def test_sample_tokens_match_oracle(orc, gpu_ctx, vocab, pad):
    """13 configurations x 2 rows, three consecutive calls carrying the states; float4 rows
    (vocab and stride multiples of 4) and scalar rows."""
    print(f"sample vocab={vocab} pad={pad}", flush=True)
    rng = np.random.default_rng(vocab + pad)
    configs = CONFIGS * 2
    states = [orc.sampler_state_new(s) for s in range(len(configs))]
    states[1] = orc.sampler_state_new(42)
    for call in range(3):
        logits = (rng.standard_normal((len(configs), vocab)) * (1.0 + call)).astype(np.float32)
        lt = padded_logits(logits, pad)
        tok, prob, new_states = run_device(gpu_ctx, lt, configs, states)
        gpu_ctx.check_faults()
        check_rows(orc, logits, configs, states, tok, prob, new_states, f"call {call}")
        states = new_states


@pytest.mark.parametrize("vocab", [64, 4096, 32000])
def test_sample_tokens_ties_and_special_values(orc, gpu_ctx, vocab):
    """Logits on a coarse grid (many equal values), with +0.0 / -0.0 and -inf mixed in: the
    set kept by streaming replacement, and the order among equal candidates, decide the
    token; both are compared exactly."""
    print(f"sample ties vocab={vocab}", flush=True)
    rng = np.random.default_rng(11)
    configs = [(1.0, k, p) for k in (2, 5, 20, 100, 1024) for p in (1.0, 0.6)]
    states = [orc.sampler_state_new(100 + i) for i in range(len(configs))]
    for call in range(4):
        logits = np.round(rng.standard_normal((len(configs), vocab)) * 2.0) / 2.0
        logits = logits.astype(np.float32)
        zero = rng.random(logits.shape) < 0.2
        logits[zero] = np.where(rng.random(zero.sum()) < 0.5, 0.0, -0.0).astype(np.float32)
        logits[rng.random(logits.shape) < 0.1] = -np.inf
        if call == 3:  # every logit equal: the earliest indices are kept
            logits[:] = 1.5
        tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
        gpu_ctx.check_faults()
        check_rows(orc, logits, configs, states, tok, prob, new_states, f"ties call {call}")
        states = new_states


@pytest.mark.parametrize("plateau", [30, 2500, 9000])
def test_sample_tokens_plateau_at_the_boundary(orc, gpu_ctx, plateau):
    """`plateau` logits share the k+1-th largest value, scattered over the row: equal
    candidates at the boundary (30), more of them than the device sorts directly (2500), more
    than one wave buffers (9000).  Which of the equal logits the reference keeps, and their
    order, follow from its replacement order; tokens and states must still match exactly."""
    print(f"sample plateau={plateau}", flush=True)
    rng = np.random.default_rng(plateau)
    vocab = 32000
    configs = [(1.0, k, p) for k in (5, 20, 300) for p in (1.0, 0.5)]
    states = [orc.sampler_state_new(7 + i) for i in range(len(configs))]
    for call in range(2):
        logits = (rng.random((len(configs), vocab)) * 3.0 - 1.0).astype(np.float32)
        for r in range(len(configs)):
            logits[r, rng.choice(vocab, plateau, replace=False)] = 2.5
            logits[r, rng.choice(vocab, 3, replace=False)] = [4.0, 3.5, 3.0]
        tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
        gpu_ctx.check_faults()
        check_rows(orc, logits, configs, states, tok, prob, new_states, f"plateau call {call}")
        states = new_states


def test_sample_tokens_c5_head_shape(orc, gpu_ctx):
    """257 rows x 128256 (the Llama-3-8B head's batch in the C5 step) under chat_default and
    greedy rows."""
    print("sample C5 head shape", flush=True)
    rng = np.random.default_rng(3)
    rows, vocab = 257, 128256
    configs = [(0.7, 20, 0.9) if r % 4 else (0.0, 1, 1.0) for r in range(rows)]
    states = [orc.sampler_state_new(r) for r in range(rows)]
    logits = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
    gpu_ctx.check_faults()
    check_rows(orc, logits, configs, states, tok, prob, new_states, "c5")


def test_sample_tokens_nan_logits(orc, gpu_ctx):
    """A NaN logit.  The greedy row takes it (total_cmp orders +NaN above +inf) with a NaN
    probability.  A sampled row never lets it in after the first k logits (NaN > min is
    false), so that row samples as the oracle does; one with the NaN among its first k logits
    cannot build a finite distribution and is reported as Runtime, its token -1 and its state
    unchanged."""
    from ferrisinfer_amd import FerrisError

    print("sample NaN logits", flush=True)
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((3, 500)).astype(np.float32)
    logits[:2, 123] = np.nan
    logits[2, 5] = np.nan
    configs = [(0.0, 1, 1.0), (0.7, 20, 0.9), (0.7, 20, 0.9)]
    states = [orc.sampler_state_new(s) for s in (1, 2, 3)]
    tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
    rt, rp, _ = orc.sample_last_token(logits[0], *configs[0], states[0])
    assert tok[0] == rt == 123 and math.isnan(prob[0]) and math.isnan(rp)
    check_rows(orc, logits[1:2], configs[1:2], states[1:2], tok[1:2], prob[1:2], new_states[1:2], "nan late")
    assert tok[2] == -1 and new_states[2] == states[2]
    with pytest.raises(FerrisError, match="finite sampling distribution"):
        gpu_ctx.check_faults()
    with pytest.raises(Exception, match="finite sampling distribution"):
        orc.sample_last_token(logits[2], *configs[2], states[2])
    gpu_ctx.check_faults()  # cleared by the previous check


def test_sample_tokens_top_k_above_1024_needs_reservation(orc):
    """On a fresh context, top_k above 1024 (after clamping to the vocabulary) is reported until
    fi_sample_reserve covers the call's rows and vocabulary, then sampled as the oracle does; a
    top_k that clamps to a vocabulary of at most 1024 needs no reservation; a vocabulary above
    2^20 cannot be reserved."""
    from ferrisinfer_amd import Context, FerrisError

    print("sample top_k reservation", flush=True)
    ctx = Context(0)
    try:
        rng = np.random.default_rng(6)
        logits = rng.standard_normal((2, 2000)).astype(np.float32)
        configs = [(0.8, 1500, 0.9), (0.8, 20, 0.9)]
        states = [orc.sampler_state_new(7), orc.sampler_state_new(8)]
        tok, _, new_states = run_device(ctx, padded_logits(logits, 0), configs, states)
        assert tok[0] == -1 and new_states[0] == states[0]
        assert tok[1] == orc.sample_last_token(logits[1], *configs[1], states[1])[0]
        with pytest.raises(FerrisError, match="top_k"):
            ctx.check_faults()
        ctx.sample_reserve(1, 2000)  # one row: the two-row call is still not covered
        tok, _, new_states = run_device(ctx, padded_logits(logits, 0), configs, states)
        assert tok[0] == -1 and new_states[0] == states[0]
        with pytest.raises(FerrisError, match="top_k"):
            ctx.check_faults()
        ctx.sample_reserve(2, 2000)
        tok, prob, new_states = run_device(ctx, padded_logits(logits, 0), configs, states)
        ctx.check_faults()
        check_rows(orc, logits, configs, states, tok, prob, new_states, "reserved")
        small = rng.standard_normal((1, 900)).astype(np.float32)
        st = [orc.sampler_state_new(9)]
        tok, prob, new_states = run_device(ctx, padded_logits(small, 0), [(0.8, 1500, 0.9)], st)
        ctx.check_faults()
        check_rows(orc, small, [(0.8, 1500, 0.9)], st, tok, prob, new_states, "clamped")
        with pytest.raises(FerrisError, match="Unsupported"):
            ctx.sample_reserve(1, (1 << 20) + 1)
    finally:
        ctx.close()


# (vocab, top_k values): the C4 vocabulary with a k just above the fast path's limit, one
# close to the vocabulary (the reference's replacement then runs over few logits) and the whole
# vocabulary (no replacement: the stable sort alone); a 32000 vocabulary with a scalar-load
# twin (32003) at mid-size k.
LARGE_K = [(151936, (2000, 150000, 151936)), (32000, (1025, 16000, 32000)), (32003, (4000, 31999))]


@pytest.mark.parametrize("vocab,ks", LARGE_K)
def test_sample_tokens_large_top_k_match_oracle(orc, gpu_ctx, vocab, ks):
    """top_k in (1024, vocab]: tokens and states exact against the oracle's replacement and
    stable sort, over two consecutive calls carrying the states, at two temperatures and three
    top-p values (NaN keeps every candidate)."""
    print(f"sample large top_k vocab={vocab} ks={ks}", flush=True)
    rng = np.random.default_rng(vocab)
    configs = [(t, k, p) for k in ks for (t, p) in ((0.7, 0.9), (1.3, 1.0), (1.0, NAN))]
    gpu_ctx.sample_reserve(len(configs), vocab)
    states = [orc.sampler_state_new(50 + i) for i in range(len(configs))]
    for call in range(2):
        logits = (rng.standard_normal((len(configs), vocab)) * (1.0 + call)).astype(np.float32)
        tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
        gpu_ctx.check_faults()
        check_rows(orc, logits, configs, states, tok, prob, new_states, f"call {call}")
        states = new_states


@pytest.mark.parametrize("vocab", [4096, 32000])
def test_sample_tokens_large_top_k_ties(orc, gpu_ctx, vocab):
    """top_k in (1024, vocab] on a coarse grid (about 25 distinct values, so nearly every draw
    lands on a value many logits share) with +0.0 / -0.0 and -inf mixed in: which of the equal
    logits the reference's replacement keeps, and their order, decide the token, and the
    device replays the replacement for them.  Then every logit equal (the earliest indices
    are kept)."""
    print(f"sample large top_k ties vocab={vocab}", flush=True)
    rng = np.random.default_rng(vocab + 1)
    configs = [(1.0, k, p) for k in (1500, 3000, vocab - 1, vocab) for p in (1.0, 0.6)]
    gpu_ctx.sample_reserve(len(configs), vocab)
    states = [orc.sampler_state_new(300 + i) for i in range(len(configs))]
    for call in range(3):
        logits = np.round(rng.standard_normal((len(configs), vocab)) * 2.0) / 2.0
        logits = logits.astype(np.float32)
        zero = rng.random(logits.shape) < 0.2
        logits[zero] = np.where(rng.random(zero.sum()) < 0.5, 0.0, -0.0).astype(np.float32)
        logits[rng.random(logits.shape) < 0.1] = -np.inf
        if call == 2:
            logits[:] = 1.5
        tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
        gpu_ctx.check_faults()
        check_rows(orc, logits, configs, states, tok, prob, new_states, f"large ties call {call}")
        states = new_states


def test_sample_tokens_large_top_k_nan(orc, gpu_ctx):
    """top_k above 1024 with a NaN logit: past the first k it never enters the list (the row
    samples as the oracle does); among the first k it makes the total NaN, reported as Runtime
    with token -1 and the state unchanged."""
    from ferrisinfer_amd import FerrisError

    print("sample large top_k NaN", flush=True)
    rng = np.random.default_rng(8)
    logits = rng.standard_normal((2, 6000)).astype(np.float32)
    logits[0, 4500] = np.nan
    logits[1, 700] = -np.nan
    configs = [(0.9, 2500, 0.95), (0.9, 2500, 0.95)]
    gpu_ctx.sample_reserve(2, 6000)
    states = [orc.sampler_state_new(11), orc.sampler_state_new(12)]
    tok, prob, new_states = run_device(gpu_ctx, padded_logits(logits, 0), configs, states)
    check_rows(orc, logits[:1], configs[:1], states[:1], tok[:1], prob[:1], new_states[:1], "nan late")
    assert tok[1] == -1 and new_states[1] == states[1]
    with pytest.raises(FerrisError, match="finite sampling distribution"):
        gpu_ctx.check_faults()
    with pytest.raises(Exception, match="finite sampling distribution"):
        orc.sample_last_token(logits[1], *configs[1], states[1])
    gpu_ctx.check_faults()


def test_sample_tokens_rejects_bad_shapes(gpu_ctx):
    import torch

    from ferrisinfer_amd import FerrisError

    z = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    f = torch.zeros(2, dtype=torch.float32, device="cuda")
    i = torch.zeros(2, dtype=torch.int32, device="cuda")
    s = torch.zeros(2, dtype=torch.int64, device="cuda")
    with pytest.raises(FerrisError, match="InvalidShape"):
        gpu_ctx.sample_tokens(z[:, :0], f, i, f, s, i, f)
