"""ctypes wrapper of the CPU oracle (liboracle.so, built from oracle.cpp).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library and the CPU
baseline leg of bench.py. Only tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg import this package; the product never does.

Every function restates reference code; the citations are in oracle.cpp.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIBRARY names another build of the oracle (the sanitizer build of
# oracle/Makefile's `sanitize` target); the default is liboracle.so here.
_LIB_PATH = os.environ.get("ORACLE_LIBRARY") or os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_set_workers.argtypes = [ctypes.c_int]
        L.orc_set_rounding.argtypes = [ctypes.c_int]
        L.orc_set_rounding_layers.argtypes = [ctypes.c_int, ctypes.c_int]
        L.orc_get_workers.restype = ctypes.c_int
        gemm_args = [ctypes.c_int] * 5 + [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.orc_sgemm.argtypes = [ctypes.c_int] + gemm_args
        L.orc_sgemm_ref.argtypes = gemm_args
        L.orc_build_sequence.argtypes = [_i32p, ctypes.c_int, ctypes.c_int32, ctypes.c_int, _i32p, _i32p, _i32p,
                                         ctypes.POINTER(ctypes.c_int)]
        L.orc_build_sequence.restype = ctypes.c_int
        L.orc_model_new.argtypes = [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int, ctypes.c_double,
                                                         ctypes.c_double, _u8p]
        L.orc_model_new.restype = ctypes.c_void_p
        L.orc_model_free.argtypes = [ctypes.c_void_p]
        L.orc_model_set.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _f32p, ctypes.c_int64]
        L.orc_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, _i32p, _i32p, _i32p, _i32p, _u8p, _i32p, _i32p,
                                  _f32p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_forward.restype = ctypes.c_int
        L.orc_forward_train.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i32p, _i32p, _u8p,
                                        _i32p, _i32p, _f32p]
        L.orc_forward_train.restype = ctypes.c_int
        L.orc_backward.argtypes = [ctypes.c_void_p, _f32p, ctypes.c_void_p, ctypes.c_int]
        L.orc_backward.restype = ctypes.c_int
        L.orc_model_zero_like.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.orc_model_get.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _f32p, ctypes.c_int64]
        L.orc_model_get.restype = ctypes.c_int
        L.orc_adamw_new.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int]
        L.orc_adamw_new.restype = ctypes.c_void_p
        L.orc_adamw_free.argtypes = [ctypes.c_void_p]
        L.orc_adamw_grad_norm.argtypes = [ctypes.c_void_p]
        L.orc_adamw_grad_norm.restype = ctypes.c_double
        L.orc_adamw_update.argtypes = [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.orc_adamw_get.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, _f32p, ctypes.c_int64]
        L.orc_adamw_get.restype = ctypes.c_int
        L.orc_layer_norm.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_void_p,
                                     ctypes.c_float]
        L.orc_gelu.argtypes = [ctypes.c_float]
        L.orc_gelu.restype = ctypes.c_float
        L.orc_gelu_grad.argtypes = [ctypes.c_float]
        L.orc_gelu_grad.restype = ctypes.c_float
        L.orc_apply_rope_inverse.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p,
                                             _f32p]
        L.orc_rope_tables.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_double, _f32p, _f32p]
        L.orc_apply_rope.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.orc_softmax_masked.argtypes = [_f32p, ctypes.c_int, ctypes.c_float, ctypes.c_void_p]
        L.orc_calibrated.argtypes = [_f64p, ctypes.c_int, ctypes.c_double, _f64p]
        L.orc_round.argtypes = [ctypes.c_double, ctypes.c_int]
        L.orc_round.restype = ctypes.c_double
        L.orc_margin_confidence.argtypes = [_f64p, ctypes.c_int]
        L.orc_margin_confidence.restype = ctypes.c_double
        L.orc_argmax.argtypes = [_f64p, ctypes.c_int]
        L.orc_argmax.restype = ctypes.c_int
        _lib = L
    return _lib


def set_workers(n: int) -> None:
    lib().orc_set_workers(int(n))


# Stage rounding switches (bit values of RND_* in oracle.cpp). Each rounds one
# stage's values to bfloat16 where a bf16 device path stores or multiplies
# them; they exist to attribute the bf16 path's logit error to its stages and
# are not part of the reference's arithmetic.
ROUND_XN, ROUND_QKV, ROUND_QK, ROUND_P, ROUND_CTX, ROUND_ACT = 1, 2, 4, 8, 16, 32
# The folded LayerNorm's operand instead of ROUND_XN's: the norm input x
# rounded (XFOLD), or x less the previous LayerNorm's row mean (XFOLDC),
# with the statistics of the unrounded rows.
ROUND_XFOLD, ROUND_XFOLDC = 256, 512


def set_rounding(mask: int, layers=(0, 1 << 30)) -> None:
    lib().orc_set_rounding(int(mask))
    lib().orc_set_rounding_layers(int(layers[0]), int(layers[1]))


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def sgemm(transA, transB, M, N, K, A, lda, B, ldb, C, ldc, accumulate, workers=None, ref=False):
    """blas.Sgemm into C (float32, modified in place)."""
    assert A.dtype == B.dtype == C.dtype == np.float32 and C.flags.c_contiguous
    L = lib()
    if ref:
        L.orc_sgemm_ref(int(transA), int(transB), M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(C), ldc,
                        int(accumulate))
    else:
        w = L.orc_get_workers() if workers is None else workers
        L.orc_sgemm(w, int(transA), int(transB), M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(C), ldc,
                    int(accumulate))
    return C


def build_sequence(ids, mask_id: int, independent: bool):
    """BuildSequence: returns (pos, opt or None, mask_pos)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n = len(ids)
    pos = np.zeros(n, np.int32)
    opt = np.zeros(n, np.int32)
    mp = np.zeros(max(n, 1), np.int32)
    has = ctypes.c_int(0)
    nm = lib().orc_build_sequence(ids, n, int(mask_id), int(bool(independent)), pos, opt, mp, ctypes.byref(has))
    return pos, (opt if has.value else None), mp[:nm].copy()


ERRORS = {-1: "malformed sequence", -2: "sequence has no options", -3: "mask position out of range",
          -4: "token id out of range", -5: "missing weight"}


class OracleModel:
    """The reference Model + Cache pair for inference (Forward with trainFrom >= Layers)."""

    def __init__(self, cfg, weights: dict):
        sliding = np.array([1 if s else 0 for s in cfg.sliding], np.uint8)
        self.cfg = cfg
        self._h = lib().orc_model_new(cfg.hidden, cfg.intermediate, cfg.heads, cfg.layers, cfg.vocab,
                                      cfg.eps, cfg.half_window, cfg.global_theta, cfg.local_theta, sliding)
        for name, arr in weights.items():
            a = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
            lib().orc_model_set(self._h, name.encode(), a, a.size)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_free(self._h)
            self._h = None

    @staticmethod
    def _flat(batch):
        seq_len = np.array([len(s.ids) for s in batch], np.int32)
        ids = np.concatenate([np.asarray(s.ids, np.int32) for s in batch]).astype(np.int32)
        pos = np.concatenate([np.asarray(s.pos, np.int32) for s in batch]).astype(np.int32)
        opt = np.concatenate([np.asarray(s.opt, np.int32) if s.opt is not None
                              else np.full(len(s.ids), -1, np.int32) for s in batch]).astype(np.int32)
        has_opt = np.array([0 if s.opt is None else 1 for s in batch], np.uint8)
        nmask = np.array([len(s.mask_pos) for s in batch], np.int32)
        mp = np.concatenate([np.asarray(s.mask_pos, np.int32) for s in batch] + [np.zeros(0, np.int32)])
        mp = np.ascontiguousarray(mp, dtype=np.int32)
        if mp.size == 0:
            mp = np.zeros(1, np.int32)
        return seq_len, ids, pos, opt, has_opt, nmask, mp

    def forward(self, batch, debug: bool = False):
        """batch: list of objects with ids, pos, opt (None = plain), mask_pos."""
        cfg = self.cfg
        seq_len, ids, pos, opt, has_opt, nmask, mp = self._flat(batch)
        R = int(nmask.sum())
        T = int(seq_len.sum())
        logits = np.zeros(max(R, 1), np.float32)
        H, L = cfg.hidden, cfg.layers
        hs = n1 = attn = None
        if debug:
            hs = np.zeros((L + 1, T, H), np.float32)
            n1 = np.zeros((L, T, H), np.float32)
            attn = np.zeros((L, T, H), np.float32)
        rc = lib().orc_forward(self._h, len(batch), seq_len, ids, pos, opt, has_opt, nmask, mp, logits,
                               _ptr(hs) if debug else None, _ptr(n1) if debug else None,
                               _ptr(attn) if debug else None)
        if rc != 0:
            raise ValueError("oracle: " + ERRORS.get(rc, str(rc)))
        if debug:
            return logits[:R], {"hs": hs, "n1": n1, "attn": attn}
        return logits[:R]

    def forward_train(self, batch, train_from: int = 0):
        """Forward(c, batch, trainFrom): keeps the activations Backward needs."""
        seq_len, ids, pos, opt, has_opt, nmask, mp = self._flat(batch)
        R = int(nmask.sum())
        logits = np.zeros(max(R, 1), np.float32)
        rc = lib().orc_forward_train(self._h, int(train_from), len(batch), seq_len, ids, pos, opt, has_opt, nmask,
                                     mp, logits)
        if rc != 0:
            raise ValueError("oracle: " + ERRORS.get(rc, str(rc)))
        self._R = R
        return logits[:R]

    def backward(self, dlogits, grads: "OracleModel", train_emb: bool = True) -> None:
        """Model.Backward: accumulates into grads (see zeros_like)."""
        dl = np.ascontiguousarray(dlogits, np.float32)
        assert dl.size == self._R
        if lib().orc_backward(self._h, dl if dl.size else np.zeros(1, np.float32), grads._h, int(train_emb)) != 0:
            raise ValueError("oracle: backward without a training forward")

    def zeros_like(self) -> "OracleModel":
        """NewLike: a model of the same configuration with every tensor zero."""
        g = OracleModel(self.cfg, {})
        lib().orc_model_zero_like(g._h, self._h)
        return g

    def get(self, name: str, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        if lib().orc_model_get(self._h, name.encode(), out, n) != 0:
            raise KeyError(name)
        return out


class OracleAdamW:
    """AdamW of internal/train/optim.go over an OracleModel and its gradients."""

    def __init__(self, model: OracleModel, grads: OracleModel, weight_decay: float, train_from: int = 0,
                 train_emb: bool = True, head_only: bool = False):
        self._model, self._grads = model, grads
        self._h = lib().orc_adamw_new(model._h, grads._h, weight_decay, train_from, int(train_emb), int(head_only))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_adamw_free(self._h)
            self._h = None

    def grad_norm(self) -> float:
        return lib().orc_adamw_grad_norm(self._h)

    def update(self, lr: float, head_lr: float, grad_scale: float = 1.0) -> None:
        lib().orc_adamw_update(self._h, lr, head_lr, grad_scale)

    def moment(self, name: str, which: int, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        if lib().orc_adamw_get(self._h, name.encode(), which, out, n) != 0:
            raise KeyError(name)
        return out


def loss_and_grad(logits, batch, targets):
    """lossAndGrad of internal/nn/nn_test.go:60-86: mean cross-entropy over
    sequences (one target option each) and dLoss/dlogits."""
    d = np.zeros(len(logits), np.float32)
    loss = 0.0
    off = 0
    nb = len(batch)
    for si, s in enumerate(batch):
        k = len(s.mask_pos)
        l = np.asarray(logits[off:off + k], np.float32)
        maxv = float(np.max(l))
        ssum = 0.0
        for v in l:
            ssum += math.exp(float(np.float32(v - np.float32(maxv))))
        for i, v in enumerate(l):
            p = math.exp(float(np.float32(v - np.float32(maxv)))) / ssum
            d[off + i] = np.float32(p) / np.float32(nb)
            if i == targets[si]:
                loss -= math.log(p) / nb
                d[off + i] = np.float32(d[off + i] - np.float32(1) / np.float32(nb))
        off += k
    return loss, d


def layer_norm(x, w, b, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    rows, dim = x.shape
    bb = np.ascontiguousarray(b, np.float32) if b is not None else None
    lib().orc_layer_norm(y, x, rows, dim, np.ascontiguousarray(w, np.float32), _ptr(bb) if bb is not None else None,
                         eps)
    return y


def gelu(x: float) -> float:
    return lib().orc_gelu(float(x))


def rope_tables(pos, head_dim, theta):
    pos = np.ascontiguousarray(pos, np.int32)
    cs = np.zeros(len(pos) * (head_dim // 2), np.float32)
    sn = np.zeros_like(cs)
    lib().orc_rope_tables(pos, len(pos), head_dim, theta, cs, sn)
    return cs, sn


def apply_rope(qkv, T, H, heads, D, cs, sn):
    lib().orc_apply_rope(qkv, T, H, heads, D, cs, sn)
    return qkv


def softmax_masked(P, n, scale, mask=None):
    m = np.ascontiguousarray(mask, np.uint8) if mask is not None else None
    lib().orc_softmax_masked(P, n, scale, _ptr(m) if m is not None else None)
    return P


def calibrated(logits, temperature):
    x = np.ascontiguousarray(logits, np.float64)
    p = np.zeros_like(x)
    lib().orc_calibrated(x, len(x), float(temperature), p)
    return p


def round_even(x, places):
    return lib().orc_round(float(x), int(places))


def margin_confidence(probs):
    return lib().orc_margin_confidence(np.ascontiguousarray(probs, np.float64), len(probs))


def argmax(x):
    return lib().orc_argmax(np.ascontiguousarray(x, np.float64), len(x))


def evaluate_question(model, kind: str, n_opt: int, ids, mask_id: int, independent: bool, temperature: float):
    """One question answered as decide.Local does it: rawLogits runs ONE
    Forward over the question's own packed sequence (local.go:182-204), then
    evalChoice / evalScore / evalNoul (local.go:264-356) post-process.
    ids are the tokenizer's Encode(PackText(...), true). Returns
    {"probs": rounded to 4 places, "choice", "confidence", "value"} with the
    conventions of dn_evaluate (choice -1 unless a Choice; value = Score
    expectation to 2 places or Noul p(first) to 4 places)."""
    out = {"probs": [], "choice": -1, "confidence": 0.0, "value": 0.0}
    if n_opt == 0:
        return out
    if kind != "noul" and n_opt == 1:  # local.go:285-287, :310-312: the model is skipped
        probs = np.ones(1)
        logits = np.zeros(1)
    else:
        ids = np.asarray(ids, np.int32)
        if len(ids) > 8192:
            raise ValueError(f"input is {len(ids)} tokens; the limit is 8192")
        pos, opt, mp = build_sequence(ids, mask_id, independent)
        if len(mp) != n_opt:
            raise ValueError("input contains the reserved [MASK] token")

        class _Seq:
            pass
        s = _Seq()
        s.ids, s.pos, s.opt, s.mask_pos = ids, pos, opt, mp
        logits = model.forward([s]).astype(np.float64)
        probs = calibrated(logits, temperature)
    if kind == "choice":
        out["choice"] = argmax(logits)
        out["confidence"] = margin_confidence(probs)
    elif kind == "score":
        expect = 0.0
        for i, p in enumerate(probs):
            expect += float(i) * p
        out["value"] = round_even(expect, 2)
        out["confidence"] = margin_confidence(probs)
    else:
        out["value"] = round_even(max(0.0, min(1.0, probs[0])), 4)
    out["probs"] = [round_even(p, 4) for p in probs]
    return out
