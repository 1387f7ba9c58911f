"""Host-side mirror of the reference's internal/nn forward interface over the
C ABI: Config (config.go), Sequence + build_sequence (forward.go:12-56) and
Engine, the device engine behind Forward (forward.go:129; gpunn/model.go:204).
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence as Seq

import numpy as np

from . import native
from .native import check, lib

# Special token ids of the ModernBERT tokenizer (internal/nn/base_test.go:34-40).
CLS_ID, SEP_ID, MASK_ID = 50281, 50282, 50284


@dataclass
class Config:
    """nn.Config (internal/nn/config.go:12-27)."""

    hidden: int
    intermediate: int
    heads: int
    layers: int
    vocab: int
    eps: float = 1e-5
    half_window: int = 64
    layer_types: List[str] = field(default_factory=list)
    global_theta: float = 160000.0
    local_theta: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def sliding(self) -> List[bool]:
        return [t == "sliding_attention" for t in self.layer_types]

    def is_sliding(self, i: int) -> bool:
        return self.layer_types[i] == "sliding_attention"


def config_from_dict(f: dict) -> Config:
    """LoadConfig (internal/nn/config.go:33-95) from a parsed HF config.json."""
    c = Config(hidden=f.get("hidden_size", 0), intermediate=f.get("intermediate_size", 0),
               heads=f.get("num_attention_heads", 0), layers=f.get("num_hidden_layers", 0),
               vocab=f.get("vocab_size", 0), eps=float(np.float32(f.get("norm_eps", 0.0))),
               half_window=f.get("local_attention", 0) // 2, layer_types=list(f.get("layer_types") or []))
    if c.eps == 0:
        c.eps = 1e-5
    if c.half_window == 0:
        c.half_window = 64
    rp = f.get("rope_parameters") or {}
    if (rp.get("full_attention") or {}).get("rope_theta", 0) > 0:
        c.global_theta = float(rp["full_attention"]["rope_theta"])
    elif f.get("global_rope_theta", 0) > 0:
        c.global_theta = float(f["global_rope_theta"])
    if (rp.get("sliding_attention") or {}).get("rope_theta", 0) > 0:
        c.local_theta = float(rp["sliding_attention"]["rope_theta"])
    elif f.get("local_rope_theta", 0) > 0:
        c.local_theta = float(f["local_rope_theta"])
    if not c.layer_types:
        every = f.get("global_attn_every_n_layers", 0) or 3
        c.layer_types = ["full_attention" if i % every == 0 else "sliding_attention" for i in range(c.layers)]
    if (c.hidden == 0 or c.heads == 0 or c.layers == 0 or len(c.layer_types) != c.layers
            or c.hidden % c.heads != 0 or c.hidden % 2 != 0):
        raise ValueError("nn: incomplete or inconsistent config")
    return c


def load_config(path: str) -> Config:
    with open(path) as fh:
        return config_from_dict(json.load(fh))


def modernbert_base() -> Config:
    """ModernBERT-base geometry: 22 layers, every 3rd global."""
    return config_from_dict({"hidden_size": 768, "intermediate_size": 1152, "num_attention_heads": 12,
                             "num_hidden_layers": 22, "vocab_size": 50368, "norm_eps": 1e-5,
                             "local_attention": 128, "global_attn_every_n_layers": 3,
                             "global_rope_theta": 160000.0, "local_rope_theta": 10000.0})


def tensor_shapes(cfg: Config) -> Dict[str, tuple]:
    """Model.Tensors() names and shapes in order (internal/nn/model.go:51-84)."""
    H, I = cfg.hidden, cfg.intermediate
    t = {"model.embeddings.tok_embeddings.weight": (cfg.vocab, H), "model.embeddings.norm.weight": (H,)}
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        if i > 0:
            t[p + "attn_norm.weight"] = (H,)
        t[p + "attn.Wqkv.weight"] = (3 * H, H)
        t[p + "attn.Wo.weight"] = (H, H)
        t[p + "mlp_norm.weight"] = (H,)
        t[p + "mlp.Wi.weight"] = (2 * I, H)
        t[p + "mlp.Wo.weight"] = (H, I)
    t.update({"model.final_norm.weight": (H,), "scorer.input_norm.weight": (H,), "scorer.input_norm.bias": (H,),
              "scorer.dense.weight": (H // 2, H), "scorer.dense.bias": (H // 2,), "scorer.norm.weight": (H // 2,),
              "scorer.norm.bias": (H // 2,), "scorer.out_proj.weight": (1, H // 2), "scorer.out_proj.bias": (1,)})
    return t


@dataclass
class Sequence:
    """nn.Sequence (internal/nn/forward.go:12-21). opt is None for plain attention."""

    ids: np.ndarray
    pos: np.ndarray
    opt: Optional[np.ndarray]
    mask_pos: np.ndarray


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def build_sequence(ids, mask_id: int, independent: bool) -> Sequence:
    """nn.BuildSequence (internal/nn/forward.go:28-56), computed by dn_build_sequence."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n = len(ids)
    pos = np.zeros(max(n, 1), np.int32)
    opt = np.zeros(max(n, 1), np.int32)
    mp = np.zeros(max(n, 1), np.int32)
    has = ctypes.c_int(0)
    nm = lib.dn_build_sequence(_ptr(ids), n, int(mask_id), int(bool(independent)), _ptr(pos), _ptr(opt), _ptr(mp),
                               ctypes.byref(has))
    if nm < 0:
        raise ValueError("dn_build_sequence: bad arguments")
    return Sequence(ids=ids, pos=pos[:n].copy(), opt=opt[:n].copy() if has.value else None,
                    mask_pos=mp[:nm].copy())


def flatten(batch: Seq[Sequence]):
    """The flattened arrays dn_forward takes (see include/decide_hip.h)."""
    seq_len = np.array([len(s.ids) for s in batch], np.int32)
    ids = np.ascontiguousarray(np.concatenate([np.asarray(s.ids, np.int32) for s in batch]), np.int32)
    pos = np.ascontiguousarray(np.concatenate([np.asarray(s.pos, np.int32) for s in batch]), np.int32)
    if all(s.opt is None for s in batch):
        opt = None
    else:
        opt = np.ascontiguousarray(np.concatenate(
            [np.asarray(s.opt, np.int32) if s.opt is not None else np.full(len(s.ids), -1, np.int32)
             for s in batch]), np.int32)
    nmask = np.array([len(s.mask_pos) for s in batch], np.int32)
    mp = np.ascontiguousarray(np.concatenate([np.asarray(s.mask_pos, np.int32) for s in batch]
                                             + [np.zeros(0, np.int32)]), np.int32)
    return seq_len, ids, pos, opt, nmask, mp


def row_tokens(batch: Seq[Sequence]) -> np.ndarray:
    """Global token index of every mask row, batch order (forward.go:180-186)."""
    out, off = [], 0
    for s in batch:
        out.extend(off + int(m) for m in s.mask_pos)
        off += len(s.ids)
    return np.array(out, np.int32)


class Engine:
    """A device-resident model: the counterpart of gpunn.Model as returned by
    train.NewInferer (internal/train/engine.go:152-167). forward(batch) has
    the contract of Model.Forward: one float32 logit per mask position, in
    batch order."""

    def __init__(self, cfg: Config, weights: Optional[Dict[str, np.ndarray]] = None, precision: str = "bf16",
                 device: int = 0, certify: float = 0.0):
        self.cfg = cfg
        self.precision = native.PRECISIONS[precision]
        h = ctypes.c_void_p()
        check(lib.dn_open(device, ctypes.byref(h)))
        self._h = h
        sl = np.array([1 if s else 0 for s in cfg.sliding], np.uint8)
        check(lib.dn_set_config(h, cfg.hidden, cfg.intermediate, cfg.heads, cfg.layers, cfg.vocab,
                                float(cfg.eps), cfg.half_window, float(cfg.global_theta), float(cfg.local_theta),
                                sl.ctypes.data_as(ctypes.c_void_p), self.precision), h)
        if certify:
            self.set_certify(certify)
        if weights is not None:
            self.load(weights)

    def load(self, weights: Dict[str, np.ndarray]) -> None:
        for name, shape in tensor_shapes(self.cfg).items():
            if name not in weights:
                raise KeyError(f"nn: missing tensor {name}")
            self.upload(name, weights[name])

    def upload(self, name: str, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        check(lib.dn_upload_tensor(self._h, name.encode(), _ptr(a), a.size), self._h)

    def upload_bf16(self, name: str, bits: np.ndarray) -> None:
        """Upload bfloat16 bit patterns (uint16), as a BF16 safetensors entry stores them."""
        a = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
        check(lib.dn_upload_tensor_bf16(self._h, name.encode(), _ptr(a), a.size), self._h)

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib.dn_close(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_stream(self, stream_handle: int) -> None:
        check(lib.dn_set_stream(self._h, ctypes.c_void_p(stream_handle)), self._h)

    def forward(self, batch: Seq[Sequence]) -> np.ndarray:
        seq_len, ids, pos, opt, nmask, mp = flatten(batch) if batch else (np.zeros(0, np.int32),) * 6
        R = int(nmask.sum()) if len(batch) else 0
        out = np.zeros(max(R, 1), np.float32)
        check(lib.dn_forward(self._h, len(batch), _ptr(seq_len), _ptr(ids), _ptr(pos), _ptr(opt), _ptr(nmask),
                             _ptr(mp if mp.size else np.zeros(1, np.int32)), _ptr(out), R), self._h)
        return out[:R]

    def forward_device(self, seq_len: np.ndarray, d_ids: int, d_pos: int, d_opt: Optional[int], nrows: int,
                       d_row_tok: int, d_logits: int) -> None:
        """Device-resident forward (pointers are raw device addresses); asynchronous."""
        seq_len = np.ascontiguousarray(seq_len, np.int32)
        check(lib.dn_forward_device(self._h, len(seq_len), _ptr(seq_len), ctypes.c_void_p(d_ids),
                                    ctypes.c_void_p(d_pos), ctypes.c_void_p(d_opt) if d_opt else None, nrows,
                                    ctypes.c_void_p(d_row_tok), ctypes.c_void_p(d_logits)), self._h)

    def forward_device_noalloc(self, seq_len: np.ndarray, d_ids: int, d_pos: int, d_opt: Optional[int], nrows: int,
                               d_row_tok: int, d_logits: int) -> None:
        """dn_forward_device_noalloc: the same forward in the library's static
        scratch array (no device allocation)."""
        sl = np.ascontiguousarray(seq_len, np.int32)
        check(lib.dn_forward_device_noalloc(self._h, len(sl), _ptr(sl), ctypes.c_void_p(d_ids), ctypes.c_void_p(d_pos),
                                            ctypes.c_void_p(d_opt) if d_opt else None, int(nrows),
                                            ctypes.c_void_p(d_row_tok), ctypes.c_void_p(d_logits)), self._h)

    def check_device_errors(self) -> None:
        check(lib.dn_check_device_errors(self._h), self._h)

    def synchronize(self) -> None:
        check(lib.dn_synchronize(self._h), self._h)

    PROBE_NAMES = ("gemm_qkv", "attention", "gemm_wo", "gemm_wi", "gemm_mlpwo")

    def set_probe(self, layer: int) -> None:
        check(lib.dn_set_probe(self._h, int(layer)), self._h)

    def read_probe(self):
        """(total ms per probed launch kind, number of forwards recorded)."""
        ms = np.zeros(5, np.float64)
        cnt = ctypes.c_int(0)
        check(lib.dn_read_probe(self._h, _ptr(ms), ctypes.byref(cnt)), self._h)
        return dict(zip(self.PROBE_NAMES, ms.tolist())), cnt.value

    def set_stream_split(self, min_tokens: int) -> None:
        """dn_set_stream_split: batches of >= min_tokens tokens run in two parts on two streams (0: off)."""
        check(lib.dn_set_stream_split(self._h, int(min_tokens)), self._h)

    def set_row_tail(self, min_tokens: int) -> None:
        """dn_set_row_tail: batches of >= min_tokens tokens (option rows at most a
        quarter of them) finish the last layer on the option rows only (0: off)."""
        check(lib.dn_set_row_tail(self._h, int(min_tokens)), self._h)

    def set_ln_fold(self, on: bool) -> None:
        """dn_set_ln_fold: bf16 and fp16 forwards of more than 1024 tokens run attn_norm
        and mlp_norm inside the GEMMs around them (default on)."""
        check(lib.dn_set_ln_fold(self._h, int(bool(on))), self._h)

    def set_small_m_loads(self, mode: int) -> None:
        """dn_set_small_m_loads: 1 operands of the small-M GEMMs through LDS (default), 0 into registers."""
        check(lib.dn_set_small_m_loads(self._h, int(mode)), self._h)

    def set_certify(self, margin: float) -> None:
        """dn_set_certify: sequences whose two best logits are closer than margin
        (or not finite) are recomputed on an fp32 twin (16-bit modes; before the
        weight uploads; 0: off)."""
        check(lib.dn_set_certify(self._h, ctypes.c_float(margin)), self._h)

    def read_certify(self):
        """dn_read_certify: (sequences checked, sequences recomputed) since the last read."""
        a, b = ctypes.c_int64(0), ctypes.c_int64(0)
        check(lib.dn_read_certify(self._h, ctypes.byref(a), ctypes.byref(b)), self._h)
        return a.value, b.value

    def mfma_calibrate(self, mode: int = 0) -> float:
        """dn_mfma_calibrate: attainable MFMA TFLOP/s (bf16: mode 0 changing operands, 1 constant;
        fp32: 2 changing, 3 constant; fp16: 4 changing, 5 constant)."""
        out = ctypes.c_double(0.0)
        check(lib.dn_mfma_calibrate(self._h, int(mode), ctypes.byref(out)), self._h)
        return out.value

    def gemm_f32(self, transA, transB, M, N, K, A, lda, B, ldb, C, ldc, accumulate) -> np.ndarray:
        """blas.Sgemm semantics on the GPU; C (float32, C-contiguous) is updated in place."""
        assert C.dtype == np.float32 and C.flags.c_contiguous
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        check(lib.dn_gemm_f32(self._h, int(transA), int(transB), M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(C), ldc,
                              int(accumulate)), self._h)
        return C

    def gemm_device(self, precision: str, M, N, K, d_A: int, d_B: int, d_C: int, accumulate=False) -> None:
        p = native.PRECISIONS[precision]
        check(lib.dn_gemm_device(self._h, p, M, N, K, ctypes.c_void_p(d_A), ctypes.c_void_p(d_B),
                                 ctypes.c_void_p(d_C), int(accumulate)), self._h)

    def gemm_device_store(self, precision: str, M, N, K, d_A: int, d_B: int, d_C: int) -> None:
        """dn_gemm_device_store: C (operand type) = A . B^T, rounded to the operand type."""
        p = native.PRECISIONS[precision]
        check(lib.dn_gemm_device_store(self._h, p, M, N, K, ctypes.c_void_p(d_A), ctypes.c_void_p(d_B),
                                       ctypes.c_void_p(d_C)), self._h)


def open_engine(cfg: Config, weights, precision="bf16", device=0) -> Engine:
    return Engine(cfg, weights, precision=precision, device=device)
