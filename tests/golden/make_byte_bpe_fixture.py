"""Writes the byte-BPE contract fixture this build's tokenizer tests read.

The data are the JSON documents the reference's own tokenizer tests hold in
memory (tests/support/text_fixture.h: the pinned Qwen3 tokenizer.json
pipeline with its vocabulary replaced by the 256 byte symbols and four
ranked merges, and Qwen3's tokenizer_config.json); they are copied out as
data files, unchanged.

    python tests/golden/make_byte_bpe_fixture.py [/root/reference]
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> None:
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    text = open(os.path.join(root, "tests", "support", "text_fixture.h"), encoding="utf-8").read()
    docs = dict(re.findall(r'inline constexpr std::string_view (\w+) =\s*R"fixture\((.*?)\)fixture";', text, re.S))
    for name, out in (("byte_bpe_json", "byte_bpe_tokenizer.json"), ("qwen3_config_json", "qwen3_tokenizer_config.json")):
        data = json.loads(docs[name])  # validates; the bytes are written as found
        assert isinstance(data, dict)
        with open(os.path.join(HERE, out), "w", encoding="utf-8") as f:
            f.write(docs[name])
        print(f"wrote {out}: {len(docs[name])} bytes")


if __name__ == "__main__":
    main()
