"""The Qwen3 chat convention (dolittle_amd/text.py) against the contract
cases of the reference's tests/core/test_qwen3_chat.cpp: formatting with
thinking enabled and disabled, the eight-ID delimiter sequence with its
expected kinds and absolute positions, chunk invariance at every split, and
position continuity.  Host code, no GPU."""
import pytest

from dolittle_amd import text as t

K = t.Kind


class ByteEcho:
    """The reference test's collaborator: protocol controls map to their
    IDs, everything else echoes bytes."""
    CONTROLS = {"<|endoftext|>": 151643, "<|im_start|>": 151644, "<|im_end|>": 151645,
                "<think>": 151667, "</think>": 151668}

    def encode(self, s):
        if s in self.CONTROLS:
            return [self.CONTROLS[s]]
        return list(s.encode("utf-8"))


IDS = [97, 151667, 98, 151668, 99, 151668, 100, 151645]
KINDS = [K.UNCLASSIFIED, K.CONTROL, K.REASONING, K.CONTROL, K.ANSWER, K.CONTROL, K.UNCLASSIFIED, K.CONTROL]


def test_formatting():
    p = t.prepare(ByteEcho(), "abc", None, thinking=True)
    assert p.formatted_utf8 == "<|im_start|>user\nabc<|im_end|>\n<|im_start|>assistant\n"
    assert p.ids == ByteEcho().encode(p.formatted_utf8) and p.stop_ids == (151645, 151643)
    d = t.prepare(ByteEcho(), "abc", "", thinking=False).formatted_utf8
    assert d.startswith("<|im_start|>system\n<|im_end|>\n") and d.endswith("<think>\n\n</think>\n\n")
    with pytest.raises(OverflowError):
        t.prepare(ByteEcho(), "x" * 100, max_bytes=64)


def test_segmentation_kinds_and_positions():
    segs = t.segment(IDS, 19, thinking=True)
    assert [s.position for s in segs] == list(range(19, 27))
    assert [s.kind for s in segs] == KINDS
    # Thinking disabled: the prompt closed the thinking section, so plain
    # IDs are answer text.
    assert [s.kind for s in t.segment([5, 6], 0, thinking=False)] == [K.ANSWER, K.ANSWER]
    # Nested opening resets; a later valid opening starts reasoning again.
    kinds = [s.kind for s in t.segment([151667, 151667, 1, 151667, 2], 0)]
    assert kinds == [K.CONTROL, K.CONTROL, K.UNCLASSIFIED, K.CONTROL, K.REASONING]


@pytest.mark.parametrize("split", range(len(IDS) + 1))
def test_chunk_invariance(split):
    cursor = t.Cursor(19, thinking=True)
    prefix = cursor.append(IDS[:split], 19)
    with pytest.raises(ValueError):
        cursor.append([], 20 + split)
    suffix = cursor.append(IDS[split:], 19 + split)
    assert [(s.position, s.kind) for s in prefix + suffix] == [(19 + i, k) for i, k in enumerate(KINDS)]


def test_tokenizer_wrapper_encodes_the_chat_prompt():
    """The chat prompt through this package's byte-level BPE on the
    reference's tokenizer fixture: the chat markers are added tokens with
    their declared IDs, and decoding returns the prompt."""
    import os
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    tok = t.ByteLevelTokenizer(open(os.path.join(golden, "byte_bpe_tokenizer.json")).read(),
                               open(os.path.join(golden, "qwen3_tokenizer_config.json")).read())
    prompt = t.format_prompt("hi", thinking=False)
    ids = tok.encode(prompt)
    assert ids[0] == t.IM_START and t.IM_END in ids and t.THINK_OPEN in ids and t.THINK_CLOSE in ids
    assert ids[1:5] == [117, 115, 101, 114]  # "user": one byte symbol each (the fixture has four merges)
    assert tok.decode(ids) == prompt
