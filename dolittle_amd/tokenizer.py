"""Byte-level BPE tokenizer for Qwen3 checkpoints (host code).

Restates the contract of src/tokenizers/byte_bpe.h:1-44 and
src/tokenizers/tokenizer.h:1-90 (make_byte_bpe, Tokenizer::encode / decode /
decode_into / max_token_bytes / contains), with the reference's own
contract cases in tests/core/test_byte_bpe.cpp:
 1. added tokens are matched on the raw input before normalization: the
    earliest match wins, the longest content at that position, then the
    lowest ID;
 2. each ordinary span between them is NFC-normalized and split with the
    tokenizer's Unicode regex, every match anchored where the last ended;
 3. each piece's UTF-8 bytes map to the ByteLevel alphabet, one symbol per
    byte;
 4. ranked merges apply lowest rank first, leftmost on a tie, never across
    pieces;
 5. the symbols resolve to vocabulary IDs, interleaved with the added-token
    IDs in input order; no BOS, EOS or padding is inserted.
Decode concatenates each ID's bytes (added tokens keep their spelling) and
records every ID's byte range; an ID outside the tokenizer decodes to an
empty range marked unmapped.  Invalid metadata or input raises
InvalidArgument, an exceeded limit LengthError.

Unicode.  The reference pins utf8proc 2.10.0 (NFC) and Oniguruma 6.9.10
(the split regex); neither is in this image.  NFC here is Python's
`unicodedata` and the split runs on the `regex` module, with the pattern's
\\s / \\S taken as the Unicode White_Space property (Oniguruma's meaning for
UTF-8 text).  For text whose code points are assigned in all of these
Unicode versions the pipeline is the same; code points assigned after the
oldest of them (Python 3.10's unicodedata is Unicode 13.0) may normalize or
classify differently.
"""
from __future__ import annotations

import heapq
import json
import unicodedata
from dataclasses import dataclass, field
from typing import Optional, Sequence, Union

import regex

from ._lib import InvalidArgument, LengthError

# The ordered split pattern of the pinned Qwen3 tokenizer.json
# (byte_bpe.cpp accepts only this pre-tokenizer).
SPLIT_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*"
                 r"|\s*[\r\n]+|\s+(?!\S)|\s+")

_BYTE_LEVEL = {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}
_SPLIT = {"type": "Split", "pattern": {"Regex": SPLIT_PATTERN}, "behavior": "Isolated", "invert": False}
_INT_MAX = (1 << 31) - 1


@dataclass(frozen=True)
class ByteBpeLimits:
    """Bounds on metadata, input text, one pre-token piece and emitted IDs
    (byte_bpe.h ByteBpeLimits); every bound must be positive."""
    max_metadata_bytes: int
    max_input_bytes: int
    max_piece_bytes: int
    max_output_tokens: int


@dataclass(frozen=True)
class TokenBytes:
    id: int
    begin: int
    end: int
    mapped: bool


@dataclass
class DecodedBytes:
    """Raw decoded bytes and each ID's [begin, end) range.  `reserve` sets the
    capacities decode_into may fill (the reference's caller-reserved
    buffers); decode_into fails before writing when they do not suffice."""
    bytes: bytes = b""
    tokens: list = field(default_factory=list)
    bytes_capacity: int = 0
    tokens_capacity: int = 0

    def reserve(self, tokens: int, nbytes: int) -> None:
        self.tokens_capacity = max(self.tokens_capacity, tokens)
        self.bytes_capacity = max(self.bytes_capacity, nbytes)


def byte_alphabet() -> list:
    """The ByteLevel alphabet: byte b maps to code point b when it is a
    printable Latin-1 character (33-126, 161-172, 174-255), the others in
    byte order to 256, 257, ..."""
    codes, extra = [], 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            codes.append(b)
        else:
            codes.append(extra)
            extra += 1
    return codes


def _require(condition: bool) -> None:
    if not condition:
        raise InvalidArgument("unsupported or invalid byte-BPE metadata")


def _parse(text: Union[str, bytes], budget: int):
    raw = text.encode() if isinstance(text, str) else bytes(text)
    if len(raw) > budget:
        raise LengthError("tokenizer metadata exceeds its budget")
    try:
        return json.loads(raw)
    except (ValueError, UnicodeDecodeError):
        raise InvalidArgument("invalid tokenizer JSON") from None


def _utf8(data: Union[str, bytes]) -> bytes:
    """The input as validated UTF-8 bytes (malformed input is rejected)."""
    if isinstance(data, str):
        try:
            return data.encode("utf-8")
        except UnicodeEncodeError:  # lone surrogates
            raise InvalidArgument("malformed UTF-8") from None
    raw = bytes(data)
    try:
        raw.decode("utf-8", "strict")
    except UnicodeDecodeError:
        raise InvalidArgument("malformed UTF-8") from None
    return raw


def _token_id(value) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise InvalidArgument("token IDs are unsigned integers")
    if value > 0xFFFFFFFF:
        raise LengthError("token ID overflow")
    return value


class ByteBpe:
    """An immutable byte-level BPE tokenizer (make_byte_bpe's result)."""

    def __init__(self, identity: str, limits: ByteBpeLimits, vocabulary: dict, decoded: dict, merges: dict,
                 alphabet: list, added: list):
        self._identity = identity
        self._limits = limits
        self._vocabulary = vocabulary      # symbol string -> ID
        self._decoded = decoded            # ID -> bytes
        self._merges = merges              # (left ID, right ID) -> (rank, output ID)
        self._alphabet = alphabet          # byte -> ID of its symbol
        self._added = added                # [(content bytes, ID)]
        self._longest = max((len(b) for b in decoded.values()), default=0)
        # \s and \S as the White_Space property, as Oniguruma reads them in
        # UTF-8 text.
        pattern = SPLIT_PATTERN.replace(r"\s", r"\p{White_Space}").replace(r"\S", r"\P{White_Space}")
        self._split = regex.compile(pattern)

    # -- Tokenizer interface (tokenizer.h:63-89)
    def identity(self) -> str:
        return self._identity

    def max_token_bytes(self) -> int:
        return self._longest

    def contains(self, token_id: int) -> bool:
        return token_id in self._decoded

    def encode(self, text: Union[str, bytes]) -> list:
        raw = _utf8(text)
        if len(raw) > self._limits.max_input_bytes:
            raise LengthError("encode byte budget")
        out: list = []
        offset = 0
        while offset < len(raw):
            selected: Optional[tuple] = None
            nearest = len(raw)
            for content, token_id in self._added:
                at = raw.find(content, offset)
                if at < 0 or at > nearest:
                    continue
                if (at < nearest or selected is None or len(content) > len(selected[0])
                        or (len(content) == len(selected[0]) and token_id < selected[1])):
                    nearest, selected = at, (content, token_id)
            self._ordinary(raw[offset:nearest], out)
            if selected is None:
                break
            self._emit(out, selected[1])
            offset = nearest + len(selected[0])
        return out

    def decode(self, ids: Sequence[int]) -> DecodedBytes:
        ids = list(ids)
        out = DecodedBytes()
        out.reserve(len(ids), self._decoded_size(ids))
        self.decode_into(ids, out)
        return out

    def decode_into(self, ids: Sequence[int], out: DecodedBytes) -> None:
        ids = list(ids)
        size = self._decoded_size(ids)
        if len(ids) > out.tokens_capacity or size > out.bytes_capacity:
            raise LengthError("decode destination capacity")
        data = bytearray()
        tokens = []
        for token_id in ids:
            start = len(data)
            piece = self._decoded.get(token_id)
            if piece is not None:
                data += piece
            tokens.append(TokenBytes(token_id, start, len(data), piece is not None))
        out.bytes = bytes(data)
        out.tokens = tokens

    # -- pipeline
    def _decoded_size(self, ids: Sequence[int]) -> int:
        if len(ids) > self._limits.max_output_tokens:
            raise LengthError("decode token budget")
        total = 0
        for token_id in ids:
            piece = self._decoded.get(token_id)
            if piece is None:
                continue
            if len(piece) > self._limits.max_input_bytes - total:
                raise LengthError("decode byte budget")
            total += len(piece)
        return total

    def _emit(self, out: list, token_id: int) -> None:
        if len(out) == self._limits.max_output_tokens:
            raise LengthError("encode token budget")
        out.append(token_id)

    def _ordinary(self, raw: bytes, out: list) -> None:
        if not raw:
            return
        text = unicodedata.normalize("NFC", raw.decode("utf-8"))
        normalized = text.encode("utf-8")
        if len(normalized) > self._limits.max_input_bytes:
            raise LengthError("normalized text budget")
        offset = 0
        while offset < len(text):
            m = self._split.match(text, offset)
            if m is None or m.end() <= offset:
                raise InvalidArgument("tokenizer regex failed to cover text")
            self._piece(text[offset:m.end()].encode("utf-8"), out)
            offset = m.end()

    def _piece(self, data: bytes, out: list) -> None:
        """Ranked merges over one piece: a doubly linked list of symbols and a
        heap of candidate pairs (rank, left position), entries checked for
        staleness when they are popped."""
        if len(data) > self._limits.max_piece_bytes:
            raise LengthError("BPE piece budget")
        n = len(data)
        if n == 0:
            return
        ids = [self._alphabet[b] for b in data]
        nxt = list(range(1, n + 1))
        prv = list(range(-1, n - 1))
        live = [True] * n
        version = [0] * n
        heap: list = []

        def offer(i: int) -> None:
            if i < 0 or i >= n or not live[i] or nxt[i] >= n:
                return
            merge = self._merges.get((ids[i], ids[nxt[i]]))
            if merge is not None:
                heapq.heappush(heap, (merge[0], i, nxt[i], version[i], merge[1]))

        for i in range(n):
            offer(i)
        while heap:
            rank, left, right, ver, output = heapq.heappop(heap)
            if not live[left] or not live[right] or nxt[left] != right or version[left] != ver:
                continue
            current = self._merges.get((ids[left], ids[right]))
            if current is None or current != (rank, output):
                continue
            ids[left] = output
            nxt[left] = nxt[right]
            version[left] += 1
            live[right] = False
            if nxt[left] < n:
                prv[nxt[left]] = left
            offer(prv[left])
            offer(left)
        i = 0
        while i < n:
            self._emit(out, ids[i])
            i = nxt[i]


def make_byte_bpe(tokenizer_json: Union[str, bytes], tokenizer_config_json: Union[str, bytes],
                  verified_source_identity: str, limits: ByteBpeLimits) -> ByteBpe:
    """Builds the tokenizer of a checkpoint's tokenizer.json and
    tokenizer_config.json (byte_bpe.h make_byte_bpe), accepting only the
    pinned Qwen3 pipeline: NFC, the Split regex then ByteLevel, a plain BPE
    model with no dropout, unknown token, byte fallback or word affixes, and
    added tokens that are not normalized or stripped and match the config's
    added_tokens_decoder."""
    _require(bool(verified_source_identity) and limits.max_metadata_bytes > 0 and limits.max_input_bytes > 0
             and limits.max_piece_bytes > 0 and limits.max_output_tokens > 0)
    _require(limits.max_input_bytes <= _INT_MAX)
    data = _parse(tokenizer_json, limits.max_metadata_bytes)
    config = _parse(tokenizer_config_json, limits.max_metadata_bytes)
    try:
        _require(data["normalizer"] == {"type": "NFC"} and data["padding"] is None and data["truncation"] is None)
        _require(data["pre_tokenizer"] == {"type": "Sequence", "pretokenizers": [_SPLIT, _BYTE_LEVEL]}
                 and data["decoder"] == _BYTE_LEVEL and data["post_processor"] == _BYTE_LEVEL)
        model = data["model"]
        _require(model["type"] == "BPE" and model["dropout"] is None and model["unk_token"] is None
                 and model["continuing_subword_prefix"] == "" and model["end_of_word_suffix"] == ""
                 and model["fuse_unk"] is False and model["byte_fallback"] is False
                 and model["ignore_merges"] is False)
        _require(config["add_bos_token"] is False and config["add_prefix_space"] is False
                 and config["clean_up_tokenization_spaces"] is False and config["split_special_tokens"] is False
                 and config["unk_token"] is None)
        codes = byte_alphabet()
        inverse = {code: b for b, code in enumerate(codes)}
        vocabulary: dict = {}
        decoded: dict = {}
        for symbol, value in model["vocab"].items():
            token_id = _token_id(value)
            _require(isinstance(symbol, str) and symbol != "" and token_id not in decoded)
            _require(all(ord(ch) in inverse for ch in symbol))
            vocabulary[symbol] = token_id
            decoded[token_id] = bytes(inverse[ord(ch)] for ch in symbol)
        alphabet = []
        for code in codes:
            _require(chr(code) in vocabulary)
            alphabet.append(vocabulary[chr(code)])
        merges: dict = {}
        for rank, merge in enumerate(model["merges"]):
            _require(isinstance(merge, list) and len(merge) == 2 and all(isinstance(m, str) for m in merge))
            left, right = merge
            _require(left in vocabulary and right in vocabulary and left + right in vocabulary)
            key = (vocabulary[left], vocabulary[right])
            _require(key not in merges)
            merges[key] = (rank, vocabulary[left + right])
        added: list = []
        seen: set = set()
        for entry in data["added_tokens"]:
            token_id = _token_id(entry["id"])
            content = entry["content"]
            _require(isinstance(content, str) and content != "" and content not in seen
                     and token_id not in decoded)
            seen.add(content)
            raw = _utf8(content)
            _require(entry["normalized"] is False and entry["lstrip"] is False and entry["rstrip"] is False
                     and entry["single_word"] is False)
            expected = {k: v for k, v in entry.items() if k != "id"}
            _require(config["added_tokens_decoder"][str(token_id)] == expected)
            added.append((raw, token_id))
            decoded[token_id] = raw
        _require(len(config["added_tokens_decoder"]) == len(added))
    except (KeyError, TypeError, AttributeError):
        raise InvalidArgument("invalid tokenizer JSON schema") from None
    identity = (f"{verified_source_identity}/byte-bpe-v1/unicodedata-{unicodedata.unidata_version}"
                f"/regex-{regex.__version__}")
    return ByteBpe(identity, limits, vocabulary, decoded, merges, alphabet, added)


def presentation(decoded: DecodedBytes) -> str:
    """The decoded bytes as text, with U+FFFD for bytes that do not form
    UTF-8 (presentation is separate from the raw bytes, tokenizer.h:21-23)."""
    return decoded.bytes.decode("utf-8", "replace")
