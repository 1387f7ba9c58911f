"""Training on the device: the counterpart of the reference's gpunn.Model
and train.gpuEngine (internal/gpunn/model.go, internal/train/engine.go:97-150)
over libdecide_hip.so's dn_* training entry points. Weights, gradients and
AdamW moments of every tensor, the scorer head included, stay on the device;
the loss and the learning-rate schedule are the caller's, as in
internal/train/trainer.go:290-330.
"""
from __future__ import annotations

import ctypes
import math
from typing import Dict, Optional, Sequence as Seq

import numpy as np

from . import native
from .native import check, lib
from .nn import Config, Engine, Sequence, _ptr, flatten, tensor_shapes

STATES = {"weight": native.DN_STATE_WEIGHT, "grad": native.DN_STATE_GRAD, "m": native.DN_STATE_M,
          "v": native.DN_STATE_V}


class TrainEngine(Engine):
    """A trainable device model. forward() is the training forward (it keeps
    the activations backward() needs); infer() is the inference forward."""

    def __init__(self, cfg: Config, weights: Optional[Dict[str, np.ndarray]] = None, precision: str = "bf16",
                 train_from: int = 0, train_emb: bool = True, device: int = 0):
        super().__init__(cfg, None, precision=precision, device=device)
        check(lib.dn_enable_training(self._h), self._h)
        self.set_trainable(train_from, train_emb)
        if weights is not None:
            self.load(weights)

    def set_trainable(self, train_from: int, train_emb: bool) -> None:
        """gpunn.(*Model).SetTrainable (internal/gpunn/model.go:155-171)."""
        check(lib.dn_set_trainable(self._h, int(train_from), int(bool(train_emb))), self._h)

    def infer(self, batch: Seq[Sequence]) -> np.ndarray:
        return Engine.forward(self, batch)

    def forward(self, batch: Seq[Sequence]) -> np.ndarray:
        seq_len, ids, pos, opt, nmask, mp = flatten(batch)
        R = int(nmask.sum())
        out = np.zeros(max(R, 1), np.float32)
        check(lib.dn_forward_train(self._h, len(batch), _ptr(seq_len), _ptr(ids), _ptr(pos), _ptr(opt), _ptr(nmask),
                                   _ptr(mp if mp.size else np.zeros(1, np.int32)), _ptr(out), R), self._h)
        return out[:R]

    def backward(self, dlogits) -> None:
        dl = np.ascontiguousarray(dlogits, np.float32)
        check(lib.dn_backward(self._h, _ptr(dl if dl.size else np.zeros(1, np.float32)), int(dl.size)), self._h)

    def zero_grad(self) -> None:
        check(lib.dn_zero_grad(self._h), self._h)

    def grad_sumsq(self) -> float:
        out = ctypes.c_double(0.0)
        check(lib.dn_grad_sumsq(self._h, ctypes.byref(out)), self._h)
        return out.value

    def grad_norm(self) -> float:
        return math.sqrt(self.grad_sumsq())

    def update(self, lr: float, head_lr: float, weight_decay: float, grad_scale: float = 1.0) -> None:
        """One AdamW step (gpunn Update + AdamW.Update on the head)."""
        check(lib.dn_adamw_step(self._h, float(lr), float(head_lr), float(weight_decay), float(grad_scale)), self._h)

    def download(self, name: str, which: str = "weight") -> np.ndarray:
        shape = tensor_shapes(self.cfg)[name]
        out = np.zeros(int(np.prod(shape)), np.float32)
        check(lib.dn_download_tensor(self._h, name.encode(), STATES[which], _ptr(out), out.size), self._h)
        return out.reshape(shape)

    def upload_state(self, name: str, which: str, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data, np.float32).reshape(-1)
        check(lib.dn_upload_state(self._h, name.encode(), STATES[which], _ptr(a), a.size), self._h)

    BWD_PROBE_NAMES = ("wgrad_qkv", "dgrad_qkv", "attention_bwd")

    def read_probe_backward(self):
        """(total ms per probed backward launch, number of backward passes recorded)."""
        ms = np.zeros(3, np.float64)
        cnt = ctypes.c_int(0)
        check(lib.dn_read_probe_backward(self._h, _ptr(ms), ctypes.byref(cnt)), self._h)
        return dict(zip(self.BWD_PROBE_NAMES, ms.tolist())), cnt.value

    def set_adam_step(self, step: int) -> None:
        check(lib.dn_set_adam_step(self._h, int(step)), self._h)


def soft_cross_entropy(logits, targets, n_items: int):
    """The trainer's loss (internal/train/trainer.go:308-321): per item,
    p = softmax(logits of its options) in float64; loss -= t_j log max(p_j,
    1e-12); dlogits = (p - t) / n_items. targets: one probability vector per
    item. Returns (summed loss, dlogits float32)."""
    dl = np.zeros(len(logits), np.float32)
    loss, off = 0.0, 0
    for t in targets:
        k = len(t)
        z = np.asarray(logits[off:off + k], np.float64)
        e = np.exp(z - z.max())
        p = e / e.sum()
        for j in range(k):
            loss -= float(t[j]) * math.log(max(p[j], 1e-12))
            dl[off + j] = np.float32((p[j] - float(t[j])) / n_items)
        off += k
    return loss, dl
