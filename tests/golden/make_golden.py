"""Writes tests/golden/lcsa_tiny.npz: a small seeded LCSA case and the oracle's selection + attention on it.

The reference ships no tensor fixtures for this path (its goldens are not committed, .gitignore:7,12), so this fixture
is produced by the oracle after the oracle is pinned (tests/test_oracle.py): the attention output is cross-checked
against the float64 brute force before it is written, and the mask has a clear top-k margin (no near-ties), so every
fp32 implementation must reproduce it bit for bit.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import lcsa as O  # noqa: E402


def main():
    heads, bh, bw, r = 2, 2, 2, 3
    s = bh * bw
    q_slices, k_slices = 1, 2
    topk = 12
    for seed in range(100):
        rng = np.random.default_rng(seed)
        q = rng.standard_normal((q_slices * s * 128, heads * 128)).astype(np.float32)
        k = rng.standard_normal((k_slices * s * 128, heads * 128)).astype(np.float32)
        v = rng.standard_normal((k_slices * s * 128, heads * 128)).astype(np.float32)
        # low-frequency structure so pooled scores are well separated
        q += 0.5 * rng.standard_normal((q_slices * s, 1, heads * 128)).repeat(128, axis=1).reshape(q.shape)
        k += 0.5 * rng.standard_normal((k_slices * s, 1, heads * 128)).repeat(128, axis=1).reshape(k.shape)
        # multiples of 1/16 in [-4, 4]: exact in bf16 too, and the fixture compresses well
        q, k, v = (np.clip(np.round(x * 16) / 16, -4, 4).astype(np.float32) for x in (q, k, v))
        local = O.local_block_mask(bh, bw, r)
        mask, probs = O.draft_block_mask_and_probs(q, k, heads, q_slices, s, local, topk)
        if O.threshold_margin(probs, q_slices, topk) > 1e-2:
            break
    out = O.block_masked_attention(q, k, v, mask, heads)
    brute = O.attention_bruteforce(q, k, v, mask, heads)
    assert O.compare(out, brute)["rel"] < 1e-12
    np.savez_compressed(os.path.join(HERE, "lcsa_tiny.npz"), q=q, k=k, v=v, local=local,
                        meta=np.array([heads, q_slices, s, topk]), mask=mask, probs=probs,
                        out=out.astype(np.float32), seed=seed)
    print("seed", seed, "margin", O.threshold_margin(probs, q_slices, topk), "kept", int(mask.sum()))


if __name__ == "__main__":
    main()
