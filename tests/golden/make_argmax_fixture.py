"""Writes tests/golden/argmax_1000.npz: the CPU oracle's logits for 1,000
requests (500 shaped like cfg2: 64-token premise + 3 options x 16; 500 like
cfg5: 40-token premise + 2 options x 12), each with its own seed, on
ModernBERT-base geometry with random_weights(seed=0), three times: with those
float32 weights (logits_f32w); with the four projection matrices rounded to
bfloat16 (round to nearest even; logits_bf16w), the values a BF16 bundle
holds and the bf16 device path multiplies; and with them rounded to IEEE
binary16 (nearest even; logits_f16w), the values the fp16 device path
multiplies; so that each device mode can be checked against the oracle on
identical weights. The oracle is the C++
restatement of the reference's Go forward and is bit-identical for any worker
count, so these logits are what the reference's CPU path gives for the same
weights and ids. The GPU test regenerates the ids from the seeds and checks
them against the stored ids.

    python tests/golden/make_argmax_fixture.py
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

N_PER_SHAPE = 500


def requests(vocab):
    """The 1,000 requests, in order: (ids, seed, shape) with seeds 10000 + i."""
    from decide_amd.nn import MASK_ID, build_sequence
    from decide_amd.synth import pack_request

    out = []
    for i in range(2 * N_PER_SHAPE):
        rng = np.random.default_rng(10000 + i)
        premise, opts = (64, [16] * 3) if i < N_PER_SHAPE else (40, [12] * 2)
        out.append(build_sequence(pack_request(rng, premise, opts, vocab), MASK_ID, True))
    return out


PROJ = ("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight")


def bf16_projection_weights(w):
    """The projection matrices rounded to bfloat16 (nearest even), widened back."""
    out = dict(w)
    for name, a in w.items():
        if name.endswith(PROJ):
            u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
            r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
            out[name] = r.astype(np.uint32).view(np.float32).reshape(a.shape)
    return out


def f16_projection_weights(w):
    """The projection matrices rounded to binary16 (nearest even), widened back."""
    return {name: (a.astype(np.float16).astype(np.float32) if name.endswith(PROJ) else a) for name, a in w.items()}


def main():
    import oracle
    from decide_amd import modernbert_base
    from decide_amd.synth import random_weights

    cfg = modernbert_base()
    batch = requests(cfg.vocab)
    oracle.set_workers(os.cpu_count() or 1)
    w = random_weights(cfg, seed=0)
    t0 = time.time()
    out = {}
    for key, weights in (("logits_f32w", w), ("logits_bf16w", bf16_projection_weights(w)),
                         ("logits_f16w", f16_projection_weights(w))):
        model = oracle.OracleModel(cfg, weights)
        out[key] = np.concatenate([model.forward(batch[i:i + 50]) for i in range(0, len(batch), 50)]).astype(
            np.float32)
    logits = out["logits_f32w"]
    ids = np.concatenate([s.ids for s in batch]).astype(np.int32)
    lens = np.array([len(s.ids) for s in batch], np.int32)
    nopt = np.array([len(s.mask_pos) for s in batch], np.int32)
    np.savez_compressed(os.path.join(HERE, "argmax_1000.npz"), ids=ids, lens=lens, nopt=nopt, **out)
    # near-ties: requests whose top two logits are within 1e-3
    gaps, off = [], 0
    for k in nopt:
        z = np.sort(logits[off:off + k])
        gaps.append(z[-1] - z[-2])
        off += k
    gaps = np.array(gaps)
    print(f"{len(batch)} requests, {int(lens.sum())} tokens, {time.time() - t0:.1f} s; "
          f"top-2 logit gap min {gaps.min():.3g}, < 1e-3: {int((gaps < 1e-3).sum())}")


if __name__ == "__main__":
    main()
