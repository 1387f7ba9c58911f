"""decide.Local answer post-processing (local.go:206-356) over dn_answer.

Given the K raw logits of one question (Model.Forward output, widened to
float64 as rawLogits does, local.go:199-203) these produce the answer fields
exactly as the reference does. Rounding is math.RoundToEven at the
reference's places.
"""
from __future__ import annotations

import ctypes

import numpy as np

from .native import check, lib


def answer(logits, temperature: float):
    """(probs, choice index, confidence) of a K-way question."""
    x = np.ascontiguousarray(np.asarray(logits, np.float32).astype(np.float64))
    p = np.zeros_like(x)
    ch = ctypes.c_int(0)
    cf = ctypes.c_double(0)
    check(lib.dn_answer(x.ctypes.data_as(ctypes.c_void_p), len(x), float(temperature),
                        p.ctypes.data_as(ctypes.c_void_p), ctypes.byref(ch), ctypes.byref(cf)))
    return p, ch.value, cf.value


def round_even(x: float, places: int) -> float:
    return lib.dn_round(float(x), int(places))


def choice_answer(keys, logits, temperature: float = 1.0) -> dict:
    """evalChoice (local.go:264-299) after the forward pass."""
    p, ch, cf = answer(logits, temperature)
    return {"choice": keys[ch], "probabilities": {k: round_even(v, 4) for k, v in zip(keys, p)}, "confidence": cf}


def score_answer(logits, temperature: float = 1.0) -> dict:
    """evalScore (local.go:301-331) after the forward pass."""
    p, _, cf = answer(logits, temperature)
    expect = float(sum(i * v for i, v in enumerate(p)))
    return {"probabilities": {str(i): round_even(v, 4) for i, v in enumerate(p)}, "score": round_even(expect, 2),
            "confidence": cf}


def noul_answer(logits, temperature: float = 1.0) -> dict:
    """evalNoul (local.go:340-356) after the forward pass: p(yes) clamped, 4 places."""
    p, _, _ = answer(logits, temperature)
    return {"noul": round_even(max(0.0, min(1.0, p[0])), 4)}
