"""Tokenizers of the byte-level API (CPU): a `tokenizers` JSON (the
reference's GPT-NeoX BPE is such a file, inference.py:171-197; a small
byte-level BPE is trained in-process here since 20B_tokenizer.json is absent)
and the byte tokenizer. The JSON tokenizer writes tokenizer_id 1 as the
reference does; the byte tokenizer writes 0."""
import numpy as np
import pytest

from krunch_amd.tokenizer import ByteTokenizer, JsonTokenizer, load_tokenizer

CORPUS = [
    "The quick brown fox jumps over the lazy dog.",
    "Lossless neural text compression with an RNN language model.",
    "naïve café — 漢字 and emoji-free unicode text, repeated: " * 3,
    "def f(x):\n    return x * 2\n",
]


def make_bpe_json(tmp_path, vocab_size: int = 400) -> str:
    """Train a byte-level BPE on a tiny corpus and save it as tokenizers JSON."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=[],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(CORPUS * 20, trainer)
    path = str(tmp_path / "bpe.json")
    tok.save(path)
    return path


def test_json_tokenizer_round_trip(tmp_path):
    t = load_tokenizer(make_bpe_json(tmp_path))
    assert isinstance(t, JsonTokenizer) and t.tokenizer_id == 1
    for text in CORPUS + ["", "unseen words: zyxwvut 12345 ~~~"]:
        ids = t.encode_bytes(text.encode())
        assert ids.dtype == np.int32 and (ids.size == 0 or (0 <= ids.min() and ids.max() < 400))
        assert t.decode_bytes(ids) == text.encode()
    # merges make common text shorter than its bytes
    assert len(t.encode_bytes(CORPUS[0].encode())) < len(CORPUS[0])


def test_json_tokenizer_replaces_invalid_utf8(tmp_path):
    """Invalid UTF-8 is decoded with replacement, as the reference's
    compress_chunk does (inference.py:203-230): such bytes do not round-trip."""
    t = load_tokenizer(make_bpe_json(tmp_path))
    raw = b"ok \xff\xfe end"
    assert t.decode_bytes(t.encode_bytes(raw)) == raw.decode("utf-8", errors="replace").encode()


def test_byte_tokenizer():
    t = load_tokenizer(None)
    assert isinstance(t, ByteTokenizer) and t.tokenizer_id == 0
    raw = bytes(range(256)) + b"\xff\x00abc"
    ids = t.encode_bytes(raw)
    assert ids.dtype == np.int32 and ids.max() == 255
    assert t.decode_bytes(ids) == raw
    with pytest.raises(ValueError):
        t.decode_bytes([256])
