"""Seeded synthetic weights and requests for the five benchmark configurations.

Weights follow InitRandom / InitHead semantics (internal/nn/model.go:133-176):
token embeddings and the four projection matrices ~ N(0, std), every norm
weight 1, scorer biases 0, scorer dense / out_proj ~ N(0, std). The normal
stream is numpy's PCG64 (``np.random.default_rng(seed)``), drawn tensor by
tensor in Model.Tensors() order; the reference's Go math/rand stream is not
reproducible here, so "identical weights" means the same arrays handed to both
the GPU engine and the CPU oracle.

Requests are packed like PackText + Encode (internal/bundle/bundle.go:81-93):
[CLS] premise... [SEP] ([MASK] option...)*K, with the last token of the last
option replaced by the trailing [SEP]. Token ids are uniform in [5, vocab)
excluding the special ids 50280-50284.
"""
from __future__ import annotations

from typing import Dict, List, Sequence as Seq

import numpy as np

from .nn import CLS_ID, MASK_ID, SEP_ID, Config, Sequence, build_sequence, tensor_shapes

SPECIAL_LO, SPECIAL_HI = 50280, 50284


def random_weights(cfg: Config, seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in tensor_shapes(cfg).items():
        if name.endswith("norm.weight"):
            out[name] = np.ones(shape, np.float32)
        elif name.endswith(".bias"):
            out[name] = np.zeros(shape, np.float32)
        else:
            a = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
            a *= np.float32(std)
            out[name] = a.reshape(shape)
    return out


def random_ids(rng: np.random.Generator, n: int, vocab: int) -> np.ndarray:
    ids = rng.integers(5, vocab, size=n, dtype=np.int64)
    bad = (ids >= SPECIAL_LO) & (ids <= SPECIAL_HI)
    while bad.any():
        ids[bad] = rng.integers(5, vocab, size=int(bad.sum()), dtype=np.int64)
        bad = (ids >= SPECIAL_LO) & (ids <= SPECIAL_HI)
    return ids.astype(np.int32)


def pack_request(rng: np.random.Generator, premise: int, option_lens: Seq[int], vocab: int,
                 cls_id=CLS_ID, sep_id=SEP_ID, mask_id=MASK_ID) -> np.ndarray:
    """[CLS] + (premise-2) ids + [SEP], then per option [MASK] + (len-1) ids;
    the final token becomes the trailing [SEP]."""
    parts = [np.array([cls_id], np.int32), random_ids(rng, premise - 2, vocab), np.array([sep_id], np.int32)]
    for ln in option_lens:
        parts.append(np.array([mask_id], np.int32))
        parts.append(random_ids(rng, ln - 1, vocab))
    ids = np.concatenate(parts).astype(np.int32)
    ids[-1] = sep_id
    return ids


# Option layouts of the SystemOne segment kinds used by cfg4: Choice K=4,
# Noul K=2, Score K=5, each segment 32 tokens.
SEGMENTS = {"choice": [8, 8, 8, 8], "noul": [16, 16], "score": [7, 7, 6, 6, 6]}
CFG4_ORDER = (["choice", "noul", "score"] * 6 + ["noul"] * 4 + ["score"] * 2)


def config_batch(name: str, vocab: int = 50368, seed: int = 0, independent: bool = True,
                 mask_id: int = MASK_ID, nseq: int = None) -> List[Sequence]:
    """The batch of one BASELINE configuration (cfg2 .. cfg5)."""
    rng = np.random.default_rng(1000 + seed)
    if name == "cfg2":
        shape = (1, 64, [16] * 3)
    elif name == "cfg3":
        shape = (64, 384, [16] * 8)
    elif name == "cfg4":
        shape = (8, 2048, [ln for kind in CFG4_ORDER for ln in SEGMENTS[kind]])
    elif name == "cfg5":
        shape = (1, 40, [12] * 2)
    else:
        raise ValueError(name)
    count, premise, opts = shape
    if nseq is not None:
        count = nseq
    return [build_sequence(pack_request(rng, premise, opts, vocab, mask_id=mask_id), mask_id, independent)
            for _ in range(count)]


def cfg4_question_groups() -> List[tuple]:
    """(kind, first logit index, K) of each question of one cfg4 sequence."""
    out, off = [], 0
    for kind in CFG4_ORDER:
        k = len(SEGMENTS[kind])
        out.append((kind, off, k))
        off += k
    return out


def systemone_call(vocab: int = 50368, seed: int = 0, state_tokens: int = 2030, instr_tokens: int = 16):
    """One SystemOne call of 24 questions over one state, as Local packs it
    (PackText + Encode: [CLS] instructions state [SEP] ([MASK] option)*K
    [SEP], bundle.go:81-93): the cfg4 question mix (Choice K=4, Noul K=2,
    Score K=5, 32 option tokens each), the same state in every question and
    16 instruction tokens of its own. Returns (kinds, n_opt, per-question
    ids) with kinds 0 = Choice, 1 = Score, 2 = Noul."""
    rng = np.random.default_rng(2000 + seed)
    state = random_ids(rng, state_tokens, vocab)
    code = {"choice": 0, "score": 1, "noul": 2}
    kinds, nopt, qids = [], [], []
    for kind in CFG4_ORDER:
        parts = [np.array([CLS_ID], np.int32), random_ids(rng, instr_tokens, vocab), state,
                 np.array([SEP_ID], np.int32)]
        for ln in SEGMENTS[kind]:
            parts += [np.array([MASK_ID], np.int32), random_ids(rng, ln - 1, vocab)]
        parts.append(np.array([SEP_ID], np.int32))
        kinds.append(code[kind])
        nopt.append(len(SEGMENTS[kind]))
        qids.append(np.concatenate(parts).astype(np.int32))
    return kinds, nopt, qids
