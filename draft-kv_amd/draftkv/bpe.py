"""Byte-level BPE tokenizers for local checkpoints (host side).

Reference: draftkv/gpt2.py:51-107 (``BPETokenizer`` over GPT-2's
``vocab.json`` + ``merges.txt``) and draftkv/llama.py:29-85 (``ByteLevelBPE``
over a HuggingFace ``tokenizer.json``). Same behaviour: text is split by the
reference's ASCII pre-tokenizer pattern, each piece's UTF-8 bytes are mapped
to GPT-2's printable byte alphabet, and adjacent symbols are merged by merge
rank, lowest first, until no ranked pair is left. ``decode`` inverts the
byte mapping (invalid UTF-8 is replaced). Enough to encode a prompt and
decode a completion for real-weight runs; nothing here touches the GPU.
"""

from __future__ import annotations

import json
import re
from pathlib import Path
from typing import Dict, List, Sequence, Union

PathLike = Union[str, Path]

# the reference's pre-tokenizer: contractions, letter / digit / other runs with
# an optional leading space, and whitespace (gpt2.py:93-95, llama.py:72-74)
_PIECES = re.compile(r"'s|'t|'re|'ve|'m|'ll|'d| ?[A-Za-z]+| ?\d+| ?[^\sA-Za-z\d]+|\s+(?!\S)|\s+")


def byte_alphabet() -> Dict[int, str]:
    """GPT-2's reversible byte -> character map: the printable Latin-1 bytes
    stand for themselves, the other 68 take the characters 256, 257, ... in
    byte order."""
    keep = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    out, extra = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return out


class _ByteBPE:
    """Shared merge loop over a vocabulary and ranked merge pairs."""

    def __init__(self, vocab: Dict[str, int], merges: Sequence[tuple]) -> None:
        self.encoder = dict(vocab)
        self.decoder = {i: t for t, i in self.encoder.items()}
        # a merge's rank is its index in the list as given (entries that are
        # not pairs keep their place), and a repeated pair keeps its last index
        self.ranks: Dict[tuple, int] = {}
        for r, pair in enumerate(merges):
            self.ranks[pair] = r
        self.b2u = byte_alphabet()
        self.u2b = {c: b for b, c in self.b2u.items()}
        self._cache: Dict[str, List[str]] = {}

    def _merge(self, piece: str) -> List[str]:
        got = self._cache.get(piece)
        if got is not None:
            return got
        syms = list(piece)
        never = 1 << 62
        while len(syms) > 1:
            ranks = [self.ranks.get((syms[i], syms[i + 1]), never) for i in range(len(syms) - 1)]
            r = min(ranks)
            if r == never:
                break
            a, b = syms[ranks.index(r)], syms[ranks.index(r) + 1]
            merged, i = [], 0
            while i < len(syms):   # every occurrence of the pair, left to right
                if i + 1 < len(syms) and syms[i] == a and syms[i + 1] == b:
                    merged.append(a + b)
                    i += 2
                else:
                    merged.append(syms[i])
                    i += 1
            syms = merged
        self._cache[piece] = syms
        return syms

    def encode(self, text: str) -> List[int]:
        ids: List[int] = []
        for piece in _PIECES.findall(text):
            mapped = "".join(self.b2u[b] for b in piece.encode("utf-8"))
            ids.extend(self.encoder[s] for s in self._merge(mapped))
        return ids

    def decode(self, ids: Sequence[int]) -> str:
        chars = "".join(self.decoder[int(i)] for i in ids)
        return bytes(self.u2b[c] for c in chars).decode("utf-8", errors="replace")


class BPETokenizer(_ByteBPE):
    """GPT-2's tokenizer from ``vocab.json`` and ``merges.txt`` (whose first
    line is a version header)."""

    def __init__(self, vocab_path: PathLike, merges_path: PathLike) -> None:
        vocab = json.loads(Path(vocab_path).read_text(encoding="utf-8"))
        lines = Path(merges_path).read_text(encoding="utf-8").split("\n")[1:]
        super().__init__(vocab, [tuple(l.split()) for l in lines if l.strip()])


class ByteLevelBPE(_ByteBPE):
    """A byte-level BPE read from a HuggingFace ``tokenizer.json`` (merges
    given as "a b" strings or [a, b] pairs)."""

    def __init__(self, path: PathLike) -> None:
        spec = json.loads(Path(path).read_text(encoding="utf-8"))
        model = spec["model"]
        super().__init__(model["vocab"], [tuple(m) if isinstance(m, list) else tuple(m.split())
                                          for m in model.get("merges", [])])
