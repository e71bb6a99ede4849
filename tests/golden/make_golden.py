"""Write tests/golden/attention_golden.json: tiny attention cases evaluated by brute force.

    python tests/golden/make_golden.py

The reference holds no golden output vectors for this path, so these are made here by an
evaluation that shares no code with the oracle: pure Python floats (IEEE float64), inputs from
random.Random, the score matrix formed entry by entry, softmax as exp(s - max) / fsum, and the
causal rule written as "key j is visible to query i iff j <= i" (the top-left tril mask of
fa2/reference.py:28-31). Query head h reads KV head h // (H_q // H_kv) (fa2/reference.py:16-19).
The oracle's naive_attention must reproduce these outputs to ~1e-12 in float64.
"""

import json
import math
import os
import random

CASES = [
    # name, B, H_q, H_kv, N_q, N_kv, D, causal, sm_scale, input scale, seed
    ("causal_mha", 1, 2, 2, 5, 5, 4, True, None, 1.0, 1),
    ("full_gqa_ragged", 2, 4, 2, 3, 7, 8, False, None, 1.0, 2),
    ("causal_mqa_scale", 1, 3, 1, 6, 6, 4, True, 0.3, 1.0, 3),
    ("causal_large_logits", 1, 2, 1, 9, 9, 16, True, None, 6.0, 4),
    ("full_single_key", 1, 2, 2, 4, 1, 4, False, None, 1.0, 5),
]


def draw(rng, shape, scale):
    if not shape:
        return rng.gauss(0.0, 1.0) * scale
    return [draw(rng, shape[1:], scale) for _ in range(shape[0])]


def brute_force(q, k, v, causal, sm_scale):
    B, H_q, N_q, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    H_kv, N_kv = len(k[0]), len(k[0][0])
    group = H_q // H_kv
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    out = []
    for b in range(B):
        heads = []
        for h in range(H_q):
            kh, vh = k[b][h // group], v[b][h // group]
            rows = []
            for i in range(N_q):
                visible = [j for j in range(N_kv) if (not causal) or j <= i]
                s = {j: scale * math.fsum(q[b][h][i][d] * kh[j][d] for d in range(D)) for j in visible}
                mx = max(s.values())
                w = {j: math.exp(s[j] - mx) for j in visible}
                z = math.fsum(w.values())
                rows.append([math.fsum(w[j] * vh[j][d] for j in visible) / z for d in range(D)])
            heads.append(rows)
        out.append(heads)
    return out


def main():
    cases = []
    for name, B, H_q, H_kv, N_q, N_kv, D, causal, sm_scale, mag, seed in CASES:
        rng = random.Random(seed)
        q = draw(rng, [B, H_q, N_q, D], mag)
        k = draw(rng, [B, H_kv, N_kv, D], mag)
        v = draw(rng, [B, H_kv, N_kv, D], 1.0)
        cases.append({"name": name, "causal": causal, "sm_scale": sm_scale,
                      "q": q, "k": k, "v": v, "out": brute_force(q, k, v, causal, sm_scale)})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_golden.json")
    with open(path, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": cases}, f)
    print(path)


if __name__ == "__main__":
    main()
