"""Writes tests/golden/seeded_inputs.json: what ferrisinfer_amd.seeded produces for the BASELINE
configurations C1-C4 at seed 0, so that another host (a Rust port of the generator, the
reference CLI) can check its regeneration of the inputs.

Stored: the generator's constants, the first draws of two streams, and per configuration the
small fields in full (lengths, block ids, arrival ticks, prompt ids of C1) and a SHA-256 of the
little-endian bytes of each large field (f32 tensors, C4 prompt ids).

Run from the repository root: python tests/golden/make_seeded_fixtures.py
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from ferrisinfer_amd import seeded, workloads as W  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "seeded_inputs.json")


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def build() -> dict:
    st = seeded.stream_states(0, 0, 4)
    first = st.copy()
    draws = [seeded.next_f32(st).tolist() for _ in range(3)]
    c2 = W.paged_decode_c2(0)
    c3 = W.prefill_c3(0)
    c1_req = W.c1_requests(0)
    c1_w = W.random_weights(W.TINY_LLAMA_C1, seed=0)
    c4_req = W.c4_requests(0)
    c4_w = W.random_weights(W.QWEN2_05B_C4, seed=0, qkv_bias=True)
    return {
        "generator": {
            "uniform": "xorshift64* of runtime/sampler.rs:55-75 (shifts 12/25/27, multiplier "
                       "0x2545F4914F6CDD1D, upper 24 bits / 2^24)",
            "stream_start": "mix64(mix64(seed ^ (tag << 32)) ^ j), zero -> 0x9e3779b97f4a7c15",
            "layout": "value i = draw i // S of stream i % S, S = min(65536, n)",
            "normal": "Box-Muller: r = sqrt(-2 ln(1 - u1)), draws 2p / 2p+1 = r cos / r sin(2 pi u2), f64",
            "integer": "lo + floor(u * (hi - lo + 1))",
            "permutation": "Fisher-Yates on stream 0, i from n-1 down to 1, j = floor(u * (i + 1))",
            "tag": "zlib CRC-32 of the field name",
            "streams": seeded.STREAMS,
        },
        "streams_seed0_tag0": {"start_states": [int(x) for x in first],
                               "draws": [[float(v) for v in d] for d in draws]},
        "C1": {
            "prompts": [[int(t) for t in p] for p, _ in c1_req],
            "max_new_tokens": [int(m) for _, m in c1_req],
            "weights_sha256": {k: sha(v) for k, v in c1_w.items()},
        },
        "C2": {
            "context_lens": [int(x) for x in c2.context_lens],
            "block_tables_sha256": sha(c2.block_tables),
            "first_block_ids": [int(x) for x in c2.block_tables[0, :16]],
            "q_sha256": sha(c2.q),
            "k_pool_sha256": sha(c2.k_pool),
            "v_pool_sha256": sha(c2.v_pool),
            "q_first": [float(x) for x in c2.q.reshape(-1)[:4]],
        },
        "C3": {
            "prompt_lens": [int(x) for x in c3.prompt_lens],
            "shared_lens": [int(x) for x in c3.shared_lens],
            "block_tables_sha256": sha(c3.block_tables),
            "q_sha256": sha(c3.q), "k_sha256": sha(c3.k_new), "v_sha256": sha(c3.v_new),
        },
        "C4": {
            "prompt_lens": [int(len(r["prompt"])) for r in c4_req],
            "max_new_tokens": [int(r["max_new_tokens"]) for r in c4_req],
            "arrival_ticks": [int(r["arrival_tick"]) for r in c4_req],
            "prompt_ids_sha256": sha(np.concatenate([r["prompt"] for r in c4_req])),
            "weights_sha256": {k: sha(v) for k, v in c4_w.items()},
        },
    }


if __name__ == "__main__":
    with open(OUT, "w") as f:
        json.dump(build(), f, indent=1)
    print(OUT)
