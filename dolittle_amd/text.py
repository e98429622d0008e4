"""The Qwen3 single-turn chat convention around the token loop (host code).

Mirrors the prompt formatting and the output segmentation of
src/text/qwen3_chat.h (algorithm in its header comment, contract cases in
tests/core/test_qwen3_chat.cpp):

- format: optional "<|im_start|>system\\n{system}<|im_end|>\\n", then
  "<|im_start|>user\\n{user}<|im_end|>\\n<|im_start|>assistant\\n", and with
  thinking disabled "<think>\\n\\n</think>\\n\\n"; nothing is trimmed or
  escaped, and the whole string is encoded with no BOS/EOS;
- stop IDs 151645 (<|im_end|>) and 151643 (<|endoftext|>);
- segmentation: thinking enabled starts unclassified, disabled starts in
  the answer; <think> (151667) from unclassified starts reasoning, </think>
  (151668) from reasoning starts the answer; any other delimiter is
  malformed and resets to unclassified; delimiters and stop IDs are control.
  A Cursor carries the state across chunks at absolute positions.

Encoding uses a tokenizer object with `encode(text) -> list[int]`; for a
checkpoint's tokenizer.json and tokenizer_config.json, `ByteLevelTokenizer`
is this package's byte-level BPE (dolittle_amd/tokenizer.py, the
restatement of src/tokenizers/byte_bpe.h).
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Optional, Sequence

IM_START, IM_END, END_OF_TEXT = 151644, 151645, 151643
THINK_OPEN, THINK_CLOSE = 151667, 151668
STOP_IDS = (IM_END, END_OF_TEXT)


class Kind(Enum):
    UNCLASSIFIED = "unclassified"
    REASONING = "reasoning"
    ANSWER = "answer"
    CONTROL = "control"


@dataclass(frozen=True)
class Segment:
    position: int
    token: int
    kind: Kind


@dataclass(frozen=True)
class Prepared:
    formatted_utf8: str
    ids: list
    stop_ids: tuple = STOP_IDS


def format_prompt(user: str, system: Optional[str] = None, thinking: bool = True) -> str:
    text = ""
    if system is not None:
        text += "<|im_start|>system\n" + system + "<|im_end|>\n"
    text += "<|im_start|>user\n" + user + "<|im_end|>\n<|im_start|>assistant\n"
    if not thinking:
        text += "<think>\n\n</think>\n\n"
    return text


def prepare(tokenizer, user: str, system: Optional[str] = None, thinking: bool = True,
            max_bytes: int = 1 << 20) -> Prepared:
    text = format_prompt(user, system, thinking)
    if len(text.encode("utf-8")) > max_bytes:
        raise OverflowError("formatted prompt exceeds its byte budget")
    return Prepared(text, list(tokenizer.encode(text)))


class Cursor:
    """Incremental segmentation; `append` must continue at the next
    absolute position, and a failed call leaves the state unchanged."""

    def __init__(self, position: int, thinking: bool = True):
        self.position = position
        self.state = Kind.UNCLASSIFIED if thinking else Kind.ANSWER

    def append(self, ids: Sequence[int], position: int) -> list:
        if position != self.position:
            raise ValueError("segment position does not continue the cursor")
        state, out = self.state, []
        for i, token in enumerate(ids):
            if token == THINK_OPEN:
                state = Kind.REASONING if state == Kind.UNCLASSIFIED else Kind.UNCLASSIFIED
                kind = Kind.CONTROL
            elif token == THINK_CLOSE:
                state = Kind.ANSWER if state == Kind.REASONING else Kind.UNCLASSIFIED
                kind = Kind.CONTROL
            elif token in STOP_IDS:
                kind = Kind.CONTROL
            else:
                kind = state
            out.append(Segment(position + i, int(token), kind))
        self.state = state
        self.position = position + len(ids)
        return out


def segment(ids: Sequence[int], position: int, thinking: bool = True) -> list:
    return Cursor(position, thinking).append(ids, position)


class ByteLevelTokenizer:
    """A checkpoint's tokenizer through this package's byte-level BPE:
    encode with no BOS/EOS, decode to text keeping added-token spellings
    (bytes that do not form UTF-8 shown as U+FFFD; `tokenizer.decode` keeps
    the raw bytes and each ID's range)."""

    def __init__(self, tokenizer_json, tokenizer_config_json, identity: str = "unverified",
                 limits: Optional["ByteBpeLimits"] = None):
        from .tokenizer import ByteBpeLimits, make_byte_bpe
        limits = limits or ByteBpeLimits(64 << 20, 1 << 24, 1 << 20, 1 << 22)
        self.tokenizer = make_byte_bpe(tokenizer_json, tokenizer_config_json, identity, limits)

    def encode(self, text: str) -> list:
        return self.tokenizer.encode(text)

    def decode(self, ids: Sequence[int]) -> str:
        from .tokenizer import presentation
        return presentation(self.tokenizer.decode(ids))
