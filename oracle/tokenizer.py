"""Pure-Python restatement of the reference's tokenizer
(internal/tokenizer/tokenizer.go), line by line, for small inputs.

TEST INFRASTRUCTURE ONLY: the checker of the library's host tokenizer
(dn_tokenizer_*). Only tests/ import it.

  parse           tokenizer.go:60-130
  encode          tokenizer.go:133-160
  split_on_tokens tokenizer.go:168-212
  pre_tokenize    tokenizer.go:214-272 (+ contraction :274-283)
  byte_to_rune    tokenizer.go:286-309
  bpe             tokenizer.go:320-365
NFC is Python's unicodedata.normalize after UAX #15's Stream-Safe Text
Process (the reference uses golang.org/x/text/unicode/norm v0.x, whose
NFC.String inserts U+034F COMBINING GRAPHEME JOINER into runs of more than
30 non-starters before normalising; unicodedata does not, so stream_safe
restates it from UAX #15 D5). Python 3.10 carries Unicode 13.0, x/text
Unicode 15.0, which differ only for code points assigned after 13.0. Text is
bytes; invalid UTF-8 follows Go: []rune makes each invalid byte one U+FFFD,
NFC passes it through.
"""
from __future__ import annotations

import json
import unicodedata

WHITE_SPACE = {0x9, 0xA, 0xB, 0xC, 0xD, 0x20, 0x85, 0xA0, 0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000} | set(
    range(0x2000, 0x200B))


def is_space(r: int) -> bool:  # unicode.IsSpace
    return r in WHITE_SPACE


def is_letter(r: int) -> bool:  # unicode.IsLetter
    return unicodedata.category(chr(r)).startswith("L")


def is_number(r: int) -> bool:  # unicode.IsNumber
    return unicodedata.category(chr(r)).startswith("N")


def go_decode(b: bytes, i: int):
    """utf8.DecodeRune at b[i:]: (rune, size); invalid -> (0xFFFD, 1)."""
    for size in (1, 2, 3, 4):
        chunk = b[i:i + size]
        if len(chunk) < size:
            break
        try:
            s = chunk.decode("utf-8")
        except UnicodeDecodeError:
            continue
        if len(s) == 1:
            return ord(s), size
    return 0xFFFD, 1


def go_runes(b: bytes):
    out, i = [], 0
    while i < len(b):
        r, n = go_decode(b, i)
        out.append(r)
        i += n
    return out


def runes_to_bytes(rs) -> bytes:
    return "".join(chr(r) for r in rs).encode("utf-8")


CGJ = "\u034f"
MAX_NON_STARTERS = 30


def nfkd_non_starters(ch: str):
    """(leading, trailing, total) counts of non-starters (canonical combining
    class != 0) in the NFKD decomposition of one character."""
    d = unicodedata.normalize("NFKD", ch)
    ns = [unicodedata.combining(c) != 0 for c in d]
    lead = next((i for i, v in enumerate(ns) if not v), len(ns))
    trail = next((i for i, v in enumerate(reversed(ns)) if not v), len(ns))
    return lead, trail, len(ns)


def stream_safe(s: str) -> str:
    """UAX #15 D5, the Stream-Safe Text Process: walking the text, keep the
    number of consecutive non-starters; before a character whose
    decomposition's leading non-starters would take it past 30, emit CGJ and
    restart the count. A character whose decomposition holds no starter adds
    all its code points to the count; any other sets it to its trailing
    non-starters."""
    out, count = [], 0
    for ch in s:
        lead, trail, total = nfkd_non_starters(ch)
        if count + lead > MAX_NON_STARTERS:
            out.append(CGJ)
            count = 0
        out.append(ch)
        count = count + total if lead == total else trail
    return "".join(out)


def nfc_run(rs) -> bytes:
    return unicodedata.normalize("NFC", stream_safe("".join(rs))).encode("utf-8")


def nfc(b: bytes) -> bytes:
    """norm.NFC.String: valid runs made stream-safe and normalised, invalid
    bytes kept (each one ends a run: x/text treats it as a starter)."""
    out, run, i = [], [], 0
    while i < len(b):
        r, n = go_decode(b, i)
        if n == 1 and b[i] >= 0x80:
            out.append(nfc_run(run))
            run = []
            out.append(b[i:i + 1])
        else:
            run.append(chr(r))
        i += n
    out.append(nfc_run(run))
    return b"".join(out)


def trim_right_space(b: bytes) -> bytes:
    rs = go_runes(b)
    # byte offsets of rune starts
    starts, i = [], 0
    while i < len(b):
        starts.append(i)
        i += go_decode(b, i)[1]
    k = len(rs)
    while k > 0 and is_space(rs[k - 1]):
        k -= 1
    return b[:starts[k]] if k < len(rs) else b


def trim_left_space(b: bytes) -> bytes:
    i = 0
    while i < len(b):
        r, n = go_decode(b, i)
        if not is_space(r):
            break
        i += n
    return b[i:]


def split_on_tokens(s: bytes, toks):
    """Leftmost-longest extraction of added tokens; (text, None) or (b"", tok)."""
    if not toks or not s:
        return [] if not s else [(s, None)]
    out, rest = [], s
    while rest:
        best, best_idx = None, -1
        for t in toks:
            c = t["content"]
            if not c:
                continue
            idx = rest.find(c)
            if idx < 0:
                continue
            if best is None or idx < best_idx or (idx == best_idx and len(c) > len(best["content"])):
                best, best_idx = t, idx
        if best is None:
            out.append((rest, None))
            break
        before = rest[:best_idx]
        if best["lstrip"]:
            before = trim_right_space(before)
        if before:
            out.append((before, None))
        out.append((b"", best))
        rest = rest[best_idx + len(best["content"]):]
        if best["rstrip"]:
            rest = trim_left_space(rest)
    return out


def contraction(rs, i):
    n = len(rs)
    if i + 1 < n and (rs[i], rs[i + 1]) in ((ord("l"), ord("l")), (ord("v"), ord("e")), (ord("r"), ord("e"))):
        return 2
    if i < n and rs[i] in (ord("s"), ord("t"), ord("m"), ord("d")):
        return 1
    return 0


def pre_tokenize(s: bytes):
    rs = go_runes(s)
    n, i, out = len(rs), 0, []
    is_o = lambda r: not is_space(r) and not is_letter(r) and not is_number(r)  # noqa: E731
    while i < n:
        start, r = i, rs[i]
        if r == ord("'") and i + 1 < n:
            ln = contraction(rs, i + 1)
            if ln > 0:
                i += 1 + ln
                out.append(runes_to_bytes(rs[start:i]))
                continue
        j = i + 1 if (r == ord(" ") and i + 1 < n) else i
        if j < n:
            c = rs[j]
            pred = is_letter if is_letter(c) else is_number if is_number(c) else is_o if is_o(c) else None
            if pred is not None:
                k = j
                while k < n and pred(rs[k]):
                    k += 1
                out.append(runes_to_bytes(rs[start:k]))
                i = k
                continue
        k = i
        while k < n and is_space(rs[k]):
            k += 1
        if k < n and k - i > 1:
            k -= 1
        out.append(runes_to_bytes(rs[start:k]))
        i = k
    return out


def _byte_to_rune():
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    m, n = {b: b for b in bs}, 0
    for b in range(256):
        if b not in m:
            m[b] = 256 + n
            n += 1
    return m


BYTE_TO_RUNE = _byte_to_rune()


class Tokenizer:
    def __init__(self, raw: bytes):
        f = json.loads(raw)
        model = f.get("model") or {}
        if model.get("type") != "BPE":
            raise ValueError(f'tokenizer: unsupported model type "{model.get("type", "")}"')
        self.vocab = dict(model.get("vocab") or {})
        self.ranks = {}
        for i, m in enumerate(model.get("merges") or []):
            if isinstance(m, list) and len(m) == 2:
                p = (m[0], m[1])
            else:
                a, sep, b = m.partition(" ")
                if not sep:
                    raise ValueError(f'tokenizer: bad merge "{m}"')
                p = (a, b)
            self.ranks.setdefault(p, i)
        self.special, self.normal = [], []
        self.cls = self.sep = self.mask = self.pad = 0
        for a in f.get("added_tokens") or []:
            t = {"id": a.get("id", 0), "content": a.get("content", "").encode("utf-8"),
                 "lstrip": bool(a.get("lstrip")), "rstrip": bool(a.get("rstrip"))}
            (self.special if a.get("special") and not a.get("normalized") else self.normal).append(t)
            c = a.get("content")
            if c == "[CLS]":
                self.cls = t["id"]
            elif c == "[SEP]":
                self.sep = t["id"]
            elif c == "[MASK]":
                self.mask = t["id"]
            elif c == "[PAD]":
                self.pad = t["id"]
        if 0 in (self.mask, self.sep, self.cls):
            raise ValueError("tokenizer: missing [CLS]/[SEP]/[MASK] added tokens")

    def bpe(self, word: bytes):
        parts = [chr(BYTE_TO_RUNE[b]) for b in word]
        while len(parts) > 1:
            best_rank, best_at = None, -1
            for i in range(len(parts) - 1):
                r = self.ranks.get((parts[i], parts[i + 1]))
                if r is not None and (best_rank is None or r < best_rank):
                    best_rank, best_at = r, i
            if best_at < 0:
                break
            parts = parts[:best_at] + [parts[best_at] + parts[best_at + 1]] + parts[best_at + 2:]
        ids = []
        for p in parts:
            if p in self.vocab:
                ids.append(self.vocab[p])
            else:
                ids.extend(self.vocab[ch] for ch in p if ch in self.vocab)
        return ids

    def encode(self, text, add_special: bool = True):
        b = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        ids = [self.cls] if add_special else []
        for seg, tok in split_on_tokens(b, self.special):
            if tok is not None:
                ids.append(tok["id"])
                continue
            for seg2, tok2 in split_on_tokens(nfc(seg), self.normal):
                if tok2 is not None:
                    ids.append(tok2["id"])
                    continue
                for w in pre_tokenize(seg2):
                    ids.extend(self.bpe(w))
        if add_special:
            ids.append(self.sep)
        return ids


def minimal_json() -> bytes:
    """tokenizer.MinimalJSON (tokenizer.go:367-395): byte-level vocabulary
    0-255, no merges, specials [CLS] 256, [SEP] 257, [MASK] 258 (lstrip),
    [PAD] 259, [UNK] 260."""
    vocab = {chr(BYTE_TO_RUNE[b]): b for b in range(256)}
    added = [{"id": 256, "content": "[CLS]", "special": True, "normalized": False, "lstrip": False},
             {"id": 257, "content": "[SEP]", "special": True, "normalized": False, "lstrip": False},
             {"id": 258, "content": "[MASK]", "special": True, "normalized": False, "lstrip": True},
             {"id": 259, "content": "[PAD]", "special": True, "normalized": False, "lstrip": False},
             {"id": 260, "content": "[UNK]", "special": True, "normalized": False, "lstrip": False}]
    return json.dumps({"added_tokens": added, "model": {"type": "BPE", "vocab": vocab, "merges": []}}).encode()
