"""Writes the committed golden fixtures from the oracle.

    python tests/golden/make_golden.py

c1_decode.npz  -- workload C1 (fp32, B1, 8 heads = 8 KV heads, d64, 4096 keys
                  in 16 chunks of 256, hot = chunks 12-15, top-2 of cold
                  chunks 0-11 by mean-key dot product).
c2_layer0.npz  -- layer 0 of workload C2 (bf16, 32/8 heads, d128, 32768 keys in
                  32 chunks of 1024, 4 planted key channels sigma 8, hot = the
                  last 8 chunks, top-4 of the 24 cold chunks).
Each holds the selected chunk indices, the raw scores, the float64 closed-form
output and LSE over hot + selected rows, the top-k score margin, and input
checksums that detect drift in the seeded generator.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as A  # noqa: E402
from oracle import scoring as S  # noqa: E402
from oracle.inputs import C1, C2, decode_inputs  # noqa: E402


def tiered_case(cfg: dict, layer_seed: int):
    x = decode_inputs(layer_seed, B=1, H=cfg["H"], H_kv=cfg["H_kv"], T=cfg["T"], D=cfg["D"],
                      dtype=cfg["dtype"], n_planted=cfg.get("n_planted", 0), sigma=cfg.get("sigma", 1.0))
    n_chunks = cfg["T"] // cfg["chunk"]
    n_cold = n_chunks - cfg["n_hot"]
    km = S.page_means(x.k, cfg["chunk"], cfg["dtype"])
    scores = S.mean_key_scores(x.q, km[:, :, :n_cold], cfg["dtype"])
    sel = S.select_chunks(x.q, km[:, :, :n_cold], np.arange(n_cold), cfg["top_k"], cfg["dtype"])
    srt = np.sort(scores.astype(np.float64))[::-1]
    margin = float(srt[cfg["top_k"] - 1] - srt[cfg["top_k"]])
    keep = np.zeros(cfg["T"], bool)
    for c in list(sel) + list(range(n_cold, n_chunks)):
        keep[c * cfg["chunk"]:(c + 1) * cfg["chunk"]] = True
    scale = 1.0 / np.sqrt(cfg["D"])
    out, lse = A.attention_f64(x.q[:, :, 0], x.k, x.v, scale=scale, keep=keep,
                               q_pos=np.array([cfg["T"] - 1]))
    chk = np.array([x.q.astype(np.float64).sum(), x.k.astype(np.float64).sum(),
                    x.v.astype(np.float64).sum(), float(x.k.reshape(-1)[12345])])
    return dict(selected=sel, scores=scores, out=out.astype(np.float32), lse=lse.astype(np.float32),
                margin=np.float64(margin), checksums=chk, planted=x.planted)


def main():
    c1 = tiered_case(C1, C1["seed"])
    np.savez_compressed(os.path.join(HERE, "c1_decode.npz"), **c1)
    print("c1 selected", c1["selected"], "margin", c1["margin"])
    c2 = tiered_case(C2, C2["seed"])
    np.savez_compressed(os.path.join(HERE, "c2_layer0.npz"), **c2)
    print("c2 selected", c2["selected"], "margin", c2["margin"], "planted", c2["planted"])


if __name__ == "__main__":
    main()
