"""decide.Local over the device engine: question types, PackText, state
formatting and one batched forward per SystemOne call.

The reference's Local.Evaluate (local.go:126-150) answers questions one at a
time, one Model.Forward each. ``Local.system_one`` lays out every question's
packed sequence in ONE batch and answers it with ``dn_evaluate``: the same
per-question checks, the same calibrated softmax, argmax and rounding
(local.go:182-356), one device forward.

``answer``/``choice_answer``/``score_answer``/``noul_answer`` are the
post-processing of one question's logits (dn_answer), exactly as the
reference rounds them (math.RoundToEven at its places).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from .native import InvalidArgument, check, lib

DN_KIND_CHOICE, DN_KIND_SCORE, DN_KIND_NOUL = 0, 1, 2

# Default option texts of a Noul without explicit criteria (local.go:333-338).
DEFAULT_YES = "Yes, condition holds true."
DEFAULT_NO = "No, condition is false."

# Local's limit on one packed sequence (local.go:29).
MAX_TOKENS = 8192


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


# ---------------------------------------------------------------------------
# Question types (types.go:22-172).

@dataclass
class Option:
    """One Choice candidate; an empty description means the key is the text (types.go:22-27)."""

    key: str
    description: str = ""


@dataclass
class Choice:
    instructions: str
    criteria: List[Option]


@dataclass
class NoulCriteria:
    true: str = ""
    false: str = ""


@dataclass
class Noul:
    instructions: str
    criteria: Optional[NoulCriteria] = None


@dataclass
class Level:
    """One Score step; examples are appended as " Examples: a, b" (types.go:114-147)."""

    what: str
    examples: List[str] = field(default_factory=list)

    def text(self) -> str:
        if not self.examples:
            return self.what.strip()
        return (self.what + " Examples: " + ", ".join(self.examples)).strip()


@dataclass
class Score:
    instructions: str
    criteria: List[Level]


def levels(*descriptions: str) -> List[Level]:
    return [Level(d) for d in descriptions]


Question = Union[Choice, Noul, Score]


@dataclass
class Calibration:
    """bundle.Calibration (internal/bundle/bundle.go:25-50)."""

    temperature: Dict[str, float] = field(default_factory=dict)
    default: float = 0.0

    def temperature_for(self, kind: str) -> float:
        t = self.temperature.get(kind, 0)
        if t > 0:
            return float(t)
        if self.default > 0:
            return float(self.default)
        return 1.0


def pack_text(state: str, instructions: str, options: Sequence[str]) -> str:
    """bundle.PackText (internal/bundle/bundle.go:81-93):
    ``<instructions> <state> [SEP] [MASK] option0 [MASK] option1 ...``."""
    prefix = (instructions + " " + state).strip() if instructions != "" else state.strip()
    return prefix + " [SEP] " + " ".join("[MASK] " + o.strip() for o in options)


def format_state(state: Any) -> str:
    """formatState (local.go:158-172): strings pass through; an object (a
    dict, or a list of (key, value) pairs) becomes "key: value" lines in its
    own key order, as a decoded JSON object keeps it (types_test.go:114);
    anything else is its string form. Values are rendered with Python's
    str(), which the reference's pyStr imitates (jsonutil.go:185-260)."""
    if isinstance(state, str):
        return state
    if isinstance(state, dict):
        state = list(state.items())
    if isinstance(state, list) and state and all(isinstance(kv, tuple) and len(kv) == 2 for kv in state):
        return "\n".join(f"{k}: {v}" for k, v in state)
    return str(state)


def _options(q: Question) -> Tuple[int, List[str], str]:
    """(kind, option texts, calibration kind) of a question, with the checks
    of evalChoice / evalScore / evalNoul (local.go:264-356)."""
    if isinstance(q, Choice):
        seen = set()
        texts = []
        for o in q.criteria:
            if o.key in seen:
                raise InvalidArgument(2, f"duplicate choice {o.key!r}")
            seen.add(o.key)
            texts.append(o.description.strip() or o.key.strip())
        return DN_KIND_CHOICE, texts, "choice"
    if isinstance(q, Score):
        return DN_KIND_SCORE, [lv.text() for lv in q.criteria], "score"
    if isinstance(q, Noul):
        yes, no = DEFAULT_YES, DEFAULT_NO
        if q.criteria is not None:
            yes = q.criteria.true.strip() or yes
            no = q.criteria.false.strip() or no
        return DN_KIND_NOUL, [yes, no], "noul"
    raise InvalidArgument(2, f"unsupported question type {type(q).__name__}")


class Local:
    """decide.Local (local.go:31-150) on a device engine.

    engine     nn.Engine with the bundle's weights resident
    encode     the bundle tokenizer's Encode(text, addSpecial=True)
               (internal/tokenizer/tokenizer.go:133-160) as a callable
    mask_id    Tokenizer.MaskID
    """

    def __init__(self, engine, encode: Callable[[str], Sequence[int]], mask_id: int, model_id: str = "decide-0.2.0",
                 independent_options: bool = True, calibration: Optional[Calibration] = None):
        self.engine = engine
        self.encode = encode
        self.mask_id = int(mask_id)
        self.model_id = model_id
        self.independent = bool(independent_options)
        self.calibration = calibration or Calibration()

    def system_one(self, state: Any, questions: Sequence[Tuple[str, Question]]) -> dict:
        """Evaluate (local.go:126-156) with one forward for all questions.
        Returns {"model", "answers": {id: answer}, "order", "usage"}."""
        state_text = format_state(state)
        kinds, nopt, qlen, temps, ids = [], [], [], [], []
        seen, q_chars, plan = set(), 0, []
        for qid, q in questions:
            if qid in seen:
                raise InvalidArgument(2, f"decide: duplicate question id {qid!r}")
            seen.add(qid)
            try:
                kind, texts, cal = _options(q)
            except InvalidArgument as e:
                raise InvalidArgument(2, f"decide: question {qid!r}: {e.message}") from None
            q_chars += len(q.instructions)
            toks: Sequence[int] = []
            if kind == DN_KIND_NOUL or len(texts) >= 2:
                toks = self.encode(pack_text(state_text, q.instructions, texts))
            kinds.append(kind)
            nopt.append(len(texts))
            qlen.append(len(toks))
            temps.append(max(self.calibration.temperature_for(cal), 1e-4))
            ids.extend(int(t) for t in toks)
            plan.append((qid, q, kind))
        nq = len(plan)
        kinds_a = np.array(kinds, np.int32)
        nopt_a = np.array(nopt, np.int32)
        qlen_a = np.array(qlen, np.int32)
        temps_a = np.array(temps, np.float64)
        ids_a = np.array(ids, np.int32)
        probs = np.zeros(max(int(nopt_a.sum()) if nq else 0, 1), np.float64)
        choice = np.zeros(max(nq, 1), np.int32)
        conf = np.zeros(max(nq, 1), np.float64)
        value = np.zeros(max(nq, 1), np.float64)
        vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        h = self.engine.handle
        rc = lib.dn_evaluate(h, nq, vp(kinds_a), vp(nopt_a), vp(qlen_a), vp(ids_a) if ids_a.size else None,
                             vp(temps_a), self.mask_id, int(self.independent), vp(probs), vp(choice), vp(conf),
                             vp(value))
        if rc:
            # Name the question by its id, as Local.Evaluate does.
            msg = lib.dn_last_error(h).decode(errors="replace")
            prefix = "decide: question "
            if msg.startswith(prefix):
                idx, _, rest = msg[len(prefix):].partition(": ")
                if idx.isdigit() and int(idx) < nq:
                    raise InvalidArgument(rc, f"decide: question {plan[int(idx)][0]!r}: {rest}")
            check(rc, h)
        answers, order, off = {}, [], 0
        for i, (qid, q, kind) in enumerate(plan):
            k = nopt[i]
            p = probs[off:off + k]
            off += k
            if kind == DN_KIND_CHOICE:
                if k == 0:
                    ans = {"choice": "", "probabilities": {}, "confidence": 0.0}
                else:
                    keys = [o.key for o in q.criteria]
                    ans = {"choice": keys[int(choice[i])], "probabilities": dict(zip(keys, p.tolist())),
                           "confidence": float(conf[i])}
            elif kind == DN_KIND_SCORE:
                legend = {str(j): lv.text() for j, lv in enumerate(q.criteria)}
                if k == 0:
                    ans = {"legend": {}, "probabilities": {}, "score": 0.0, "confidence": 0.0}
                else:
                    ans = {"legend": legend, "probabilities": {str(j): v for j, v in enumerate(p.tolist())},
                           "score": float(value[i]), "confidence": float(conf[i])}
            else:
                ans = {"noul": float(value[i])}
            answers[qid] = ans
            order.append(qid)
        usage = {"input_tokens": max(1, len(state_text) // 4) + max(1, q_chars // 4), "output_tokens": len(answers)}
        return {"model": self.model_id, "answers": answers, "order": order, "usage": usage}
