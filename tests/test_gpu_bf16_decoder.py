"""GPU parity of the bf16-weight decoder step (ferrisinfer_amd.bf16_decoder) at the C5
(Llama-3-8B) layer shape: one decoder layer over a mixed step of decode rows and a prefill chunk
on a bf16 KV pool, against the oracle's restatement of the reference decoder block
(runtime/reference.rs:163-370: rms_norm, linear, rope, cached-prefixed attention, SwiGLU,
residual adds) with the same bf16 weights widened to f32 and K/V stored as bf16.

Checks:
* the attention stage on the step's own inputs: the oracle's cached-prefixed attention on the
  step's rotated queries and the pool contents after the append (prefix rows + the appended
  rows, read back through the block tables) matches the decode rows within 1e-4 (f32 math) and
  the prefill chunk within 1e-2 (bf16 MFMA: queries and probabilities rounded to bf16);
* the whole layer within the bf16-storage bound 2e-2 normwise of the reference semantics (f32
  activations), and within 5e-3 of the oracle run with the projection inputs and the appended
  K/V rounded to bf16 as the GPU path does.  That second bound cannot be tight: the two
  computations carry ~1e-4 different f32 error into each bf16 rounding, which moves the elements
  near a rounding boundary by a whole bf16 step (2^-8 relative);
* greedy ids exact outside near ties.
The head uses a 4096-token vocabulary to keep the oracle's head product small; its shape is
covered by tests/test_gpu_bf16_gemm.py.
"""
import numpy as np
import pytest

from conftest import normwise_error

pytestmark = pytest.mark.gpu


def test_bf16_decoder_layer_matches_reference(orc):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from ferrisinfer_amd import Context
    from ferrisinfer_amd.bf16_decoder import LLAMA3_8B_C5, Bf16Decoder, build_step_batch

    cfg = dict(LLAMA3_8B_C5, layers=1, vocab=4096)
    h, f, v, hq, hkv = cfg["hidden"], cfg["intermediate"], cfg["vocab"], cfg["heads"], cfg["kv_heads"]
    d = h // hq
    bs, eps, theta = 16, cfg["eps"], cfg["theta"]
    rng = np.random.default_rng(5)
    decode_ctx = [37, 1, 70, 16, 129]          # includes the new token
    prefill = [(16, 19)]                       # 19 new tokens after a 16-token cached prefix
    lens = decode_ctx + [p + n for p, n in prefill]
    num_blocks = sum((n + bs - 1) // bs for n in lens) + 3
    nd, t = len(decode_ctx), len(decode_ctx) + sum(n for _, n in prefill)
    print(f"bf16 decoder layer: decode {decode_ctx}, prefill {prefill}", flush=True)

    def wbits(*shape):
        return orc.f32_to_bf16((rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32))

    W = dict(wq=wbits(h, h), wk=wbits(h, hkv * d), wv=wbits(h, hkv * d), wo=wbits(h, h),
             w1=wbits(h, f), w2=wbits(f, h), w3=wbits(h, f))
    head = wbits(v, h)
    attn_norm = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    ffn_norm = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    final_norm = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    pool_bits = orc.f32_to_bf16(rng.standard_normal((2, num_blocks, hkv, bs, d), dtype=np.float32))
    x = (rng.standard_normal((t, h), dtype=np.float32) * np.float32(0.5)).astype(np.float32)

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    ctx = Context(0)
    dec = Bf16Decoder(ctx, cfg, num_blocks, bs, max_tokens=t, max_last_rows=len(lens))
    dec.set_layer(*(dev(W[k].view(np.int16)) for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")),
                  dev(attn_norm), dev(ffn_norm))
    dec.set_head(dev(final_norm), dev(head.view(np.int16)))
    dec.k_pools[0].copy_(dev(pool_bits[0].view(np.int16)))
    dec.v_pools[0].copy_(dev(pool_bits[1].view(np.int16)))
    batch, tables = build_step_batch(decode_ctx, prefill, bs, num_blocks, seed=3)
    out_h = dec.step(dev(x), batch, head=False).cpu().numpy()
    got_q = dec.q[:t].cpu().numpy()        # layer 0's rotated queries
    got_attn = dec.attn[:t].cpu().numpy()  # layer 0's attention output
    got_pool = np.stack([orc.bf16_to_f32(dec.k_pools[0].cpu().numpy().view(np.uint16)),
                         orc.bf16_to_f32(dec.v_pools[0].cpu().numpy().view(np.uint16))])
    tok, prob = dec.step(dev(x), batch)
    tok, prob = tok.cpu().numpy(), prob.cpu().numpy()
    ctx.check_faults()
    ctx.close()

    Wf = {k: orc.bf16_to_f32(b) for k, b in W.items()}
    pool = orc.bf16_to_f32(pool_bits)
    starts = [c - 1 for c in decode_ctx] + [p for p, _ in prefill]      # cached tokens per sequence
    news = [1] * nd + [n for _, n in prefill]
    rows = np.cumsum([0] + news)

    inter = {}

    def layer(xin, round_inputs):
        rnd = (lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a))) if round_inputs else (lambda a: a)
        normed = orc.rms_norm(xin, attn_norm, eps)
        q = orc.linear_with_bias(rnd(normed), Wf["wq"]).reshape(t, hq, d)
        k = orc.linear_with_bias(rnd(normed), Wf["wk"]).reshape(t, hkv, d)
        vv = orc.linear_with_bias(rnd(normed), Wf["wv"]).reshape(t, hkv, d)
        attn = np.zeros((t, hq, d), np.float32)
        qrot = np.zeros((t, hq, d), np.float32)
        for s in range(len(lens)):
            r0, r1, start = rows[s], rows[s + 1], starts[s]
            qs, ks = orc.rope(q[r0:r1], k[r0:r1], start, d, theta)
            qrot[r0:r1] = qs
            ks = orc.bf16_to_f32(orc.f32_to_bf16(ks))         # appended to the bf16 pool
            vs = orc.bf16_to_f32(orc.f32_to_bf16(vv[r0:r1]))
            ids = [tables[s][p // bs] for p in range(start)]
            offs = [p % bs for p in range(start)]
            ck = pool[0][ids, :, offs, :] if start else np.zeros((0, hkv, d), np.float32)
            cv = pool[1][ids, :, offs, :] if start else np.zeros((0, hkv, d), np.float32)
            attn[r0:r1] = orc.cached_prefixed_causal_attention(qs, ck, cv, start, ks, vs)
        if round_inputs:
            inter.update(q=qrot, attn=attn)
        h1 = orc.add(xin, orc.linear_with_bias(rnd(attn.reshape(t, h)), Wf["wo"]))
        n2 = orc.rms_norm(h1, ffn_norm, eps)
        up = orc.linear_with_bias(rnd(n2), Wf["w1"])
        gate = orc.linear_with_bias(rnd(n2), Wf["w3"])
        act = orc.mul(up, orc.silu(gate))
        return orc.add(h1, orc.linear_with_bias(rnd(act), Wf["w2"]))

    # attention stage on the step's own inputs
    for s in range(len(lens)):
        r0, r1, start = rows[s], rows[s + 1], starts[s]
        ids = [tables[s][p // bs] for p in range(lens[s])]
        offs = [p % bs for p in range(lens[s])]
        kk, vv = got_pool[0][ids, :, offs, :], got_pool[1][ids, :, offs, :]
        want = orc.cached_prefixed_causal_attention(got_q[r0:r1], kk[:start], vv[:start], start,
                                                    kk[start:], vv[start:])
        assert normwise_error(got_attn[r0:r1], want) <= (1e-4 if s < nd else 1e-2), s

    ref = layer(x, round_inputs=False)
    tight = layer(x, round_inputs=True)
    err_ref, err_tight = normwise_error(out_h, ref), normwise_error(out_h, tight)
    err_q, err_attn = normwise_error(got_q, inter["q"]), normwise_error(got_attn, inter["attn"])
    print(f"q {err_q:.2e} attn {err_attn:.2e} (decode rows {normwise_error(got_attn[:nd], inter['attn'][:nd]):.2e}, "
          f"prefill rows {normwise_error(got_attn[nd:], inter['attn'][nd:]):.2e}); "
          f"hidden: vs reference {err_ref:.2e}, vs bf16-input oracle {err_tight:.2e}", flush=True)
    assert err_ref <= 2e-2
    assert err_tight <= 5e-3

    last = [rows[s + 1] - 1 for s in range(len(lens))]
    fin = orc.rms_norm(tight[last], final_norm, eps)
    fin_r = orc.bf16_to_f32(orc.f32_to_bf16(fin))
    headf = orc.bf16_to_f32(head)
    logits = fin_r.astype(np.float64) @ headf.T.astype(np.float64)
    for i in range(len(lens)):
        top2 = np.sort(logits[i])[-2:]
        if top2[1] - top2[0] < 1e-2 * max(1.0, abs(top2[1])):
            continue  # near tie at bf16 resolution
        ridx, _ = orc.matmul_rhs_transposed_argmax(fin_r[i:i + 1], headf)
        assert int(tok[i]) == ridx, i


def test_bf16_decoder_activation_handover_bit_identical():
    """Two C5-shaped layers over the same mixed step with the projections' inputs handed over as
    bf16 bits (the default) and as f32: the GEMMs round f32 inputs to bf16 by the same rule, so
    the final hidden rows, the appended K/V pools, tokens and probabilities agree bit for bit."""
    import torch

    from ferrisinfer_amd import Context
    from ferrisinfer_amd.bf16_decoder import LLAMA3_8B_C5, Bf16Decoder, build_step_batch

    import oracle

    cfg = dict(LLAMA3_8B_C5, layers=2, vocab=4096)
    h, f, v, hq, hkv = cfg["hidden"], cfg["intermediate"], cfg["vocab"], cfg["heads"], cfg["kv_heads"]
    d = h // hq
    bs = 16
    rng = np.random.default_rng(11)
    decode_ctx = [300, 5, 1030]
    prefill = [(64, 200)]
    lens = decode_ctx + [p + n for p, n in prefill]
    num_blocks = sum((n + bs - 1) // bs for n in lens) + 2
    t = len(decode_ctx) + sum(n for _, n in prefill)
    print(f"bf16 decoder handover: decode {decode_ctx}, prefill {prefill}", flush=True)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731

    def wbits(*shape):
        return dev(oracle.f32_to_bf16((rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))).view(np.int16))

    layers = [[wbits(h, h), wbits(h, hkv * d), wbits(h, hkv * d), wbits(h, h), wbits(h, f), wbits(f, h), wbits(h, f),
               dev((1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)),
               dev((1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32))] for _ in range(2)]
    final_norm = dev((1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32))
    head = wbits(v, h)
    pools = dev(oracle.f32_to_bf16(rng.standard_normal((4, num_blocks, hkv, bs, d), dtype=np.float32)).view(np.int16))
    x = dev((rng.standard_normal((t, h), dtype=np.float32) * np.float32(0.5)).astype(np.float32))
    ctx = Context(0)
    runs = []
    for b16 in (True, False):
        dec = Bf16Decoder(ctx, cfg, num_blocks, bs, max_tokens=t, max_last_rows=len(lens), bf16_activations=b16)
        for lw in layers:
            dec.set_layer(*lw)
        dec.set_head(final_norm, head)
        for i in range(2):
            dec.k_pools[i].copy_(pools[2 * i])
            dec.v_pools[i].copy_(pools[2 * i + 1])
        batch, _ = build_step_batch(decode_ctx, prefill, bs, num_blocks, seed=4)
        hid = dec.step(x, batch, head=False).clone()
        tok, prob = dec.step(x, batch)
        runs.append((hid, tok.clone(), prob.clone(), [p.clone() for p in dec.k_pools + dec.v_pools]))
        del dec
    ctx.check_faults()
    ctx.close()
    (h16, t16, p16, k16), (h32, t32, p32, k32) = runs
    assert torch.equal(h16, h32)
    assert torch.equal(t16, t32) and torch.equal(p16, p32)
    assert all(torch.equal(a, b) for a, b in zip(k16, k32))
