"""The host tokenizer of libdecide_hip.so (dn_tokenizer_*): ModernBERT's
byte-level BPE as internal/tokenizer/tokenizer.go implements it (NFC, the
GPT-2 pre-tokenizer, added tokens, [CLS] $A [SEP])."""
from __future__ import annotations

import ctypes
from typing import List

import numpy as np

from .native import DN_INVALID_ARG, check, lib


def _buf(data: bytes):
    return ctypes.cast(ctypes.c_char_p(data), ctypes.c_void_p)


class Tokenizer:
    """tokenizer.Tokenizer: parse(tokenizer.json bytes) or load(path)."""

    def __init__(self, handle: ctypes.c_void_p):
        self._h = handle
        ids = [ctypes.c_int32(0) for _ in range(4)]
        check(lib.dn_tokenizer_special_ids(self._h, *[ctypes.byref(x) for x in ids]))
        self.cls_id, self.sep_id, self.mask_id, self.pad_id = (x.value for x in ids)

    @classmethod
    def parse(cls, raw: bytes) -> "Tokenizer":
        h = ctypes.c_void_p()
        check(lib.dn_tokenizer_parse(_buf(raw), len(raw), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def load(cls, path: str) -> "Tokenizer":
        with open(path, "rb") as fh:
            return cls.parse(fh.read())

    def encode(self, text: str, add_special: bool = True) -> List[int]:
        raw = text.encode("utf-8", errors="surrogatepass") if isinstance(text, str) else bytes(text)
        cap = len(raw) + 2
        while True:
            out = np.zeros(max(cap, 1), np.int32)
            n = ctypes.c_int64(0)
            rc = lib.dn_tokenize(self._h, _buf(raw), len(raw), int(add_special), out.ctypes.data_as(ctypes.c_void_p),
                                 cap, ctypes.byref(n))
            if rc == DN_INVALID_ARG and n.value > cap:
                cap = n.value
                continue
            check(rc)
            return out[:n.value].tolist()

    def count(self, text: str) -> int:
        """Tokenizer.Count: ids without the special tokens."""
        return len(self.encode(text, add_special=False))

    def __call__(self, text: str) -> List[int]:
        return self.encode(text, True)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib.dn_tokenizer_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pretokenize(text) -> List[str]:
    """preTokenize (tokenizer.go:214-272) through dn_pretokenize: the pieces."""
    raw = text.encode("utf-8") if isinstance(text, str) else bytes(text)
    cap = len(raw) + 1
    ends = np.zeros(cap, np.int64)
    n = ctypes.c_int64(0)
    check(lib.dn_pretokenize(_buf(raw), len(raw), ends.ctypes.data_as(ctypes.c_void_p), cap, ctypes.byref(n)))
    # Offsets index the text with each invalid byte as U+FFFD (Go's []rune).
    fixed = _one_fffd_per_invalid_byte(raw)
    out, prev = [], 0
    for e in ends[:n.value]:
        out.append(fixed[prev:int(e)].decode("utf-8"))
        prev = int(e)
    return out


def _one_fffd_per_invalid_byte(raw: bytes) -> bytes:
    out, i = [], 0
    while i < len(raw):
        for size in (1, 2, 3, 4):
            try:
                if len(raw[i:i + size]) == size and len(raw[i:i + size].decode("utf-8")) == 1:
                    out.append(raw[i:i + size])
                    i += size
                    break
            except UnicodeDecodeError:
                continue
        else:
            out.append("\ufffd".encode("utf-8"))
            i += 1
    return b"".join(out)


def nfc(text) -> bytes:
    """NFC through dn_nfc (bytes in, bytes out; invalid bytes pass through)."""
    raw = text.encode("utf-8") if isinstance(text, str) else bytes(text)
    cap = 3 * len(raw) + 16
    out = ctypes.create_string_buffer(cap)
    n = ctypes.c_int64(0)
    check(lib.dn_nfc(_buf(raw), len(raw), ctypes.cast(out, ctypes.c_void_p), cap, ctypes.byref(n)))
    return out.raw[:n.value]
