"""The .mia tokenizer and chat text of the serve path (host/tokenizer.c), on the
CPU: ids equal to the reference's own tokenizer (src/tokenizer/bpe.c,
tests/golden/tokenizer.npz from oracle/_ref) for 46 texts under four
vocabularies, the reference's unit tests (tests/test_tokenizer.c), decoding
round trips, blob validation, the chat-turn text (src/model/runtime.c:84-95)
and the serve program's command-line errors."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

import motoria_amd as M
import mia_writer as MW

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def golden():
    g = np.load(os.path.join(GOLDEN, "tokenizer.npz"))
    return g, json.loads(str(g["manifest"]))


def test_ids_equal_the_reference(golden):
    g, man = golden
    toks = {}
    for c in man["cases"]:
        v = c["vocab"]
        if v not in toks:
            toks[v] = M.Bpe(g["blob_" + v].tobytes())
        if c["key"] is None:
            assert toks[v].encode(c["text"], max_ids=c["max"]) is None, (v, "overflow")
            continue
        want = g["ids_" + c["key"]].tolist()
        assert toks[v].encode(c["text"]) == want, (v, c["text"][:40])
    assert len(toks) == 4


def test_chat_text_equals_the_reference(golden):
    _, man = golden
    for c in man["chat"]:
        assert M.chat_turn_text(c["user"], c["think"], c["continuing"]) == c["text"]


def unit_tokenizer():
    # tests/test_tokenizer.c:24-39 of the reference
    pieces = [b"a", b"b", b"c", b" ", b"ab", b"abc", b" abc", b"<|im_end|>", b"!", b"x"]
    return M.Bpe(MW.mtk1_blob(pieces, [(0, 1, 4), (4, 2, 5), (3, 5, 6)], specials=(7,),
                              im_end=7))


def test_reference_unit_cases():
    t = unit_tokenizer()
    assert t.encode("abc abc") == [5, 6]             # merges follow rank order
    assert t.encode("ba") == [1, 0]                  # unmergeable bytes stay single
    assert t.encode("abc<|im_end|>abc") == [5, 7, 5]  # specials match verbatim
    assert t.encode("abc!abc") == [5, 8, 5]          # punctuation splits from words
    text = b"abc abc!<|im_end|>"
    assert b"".join(t.piece(i) for i in t.encode(text)) == text
    assert t.is_stop(7) and not t.is_stop(5) and t.im_start() == -1
    assert t.piece(-1) == b"" and t.piece(10) == b""


def test_decode_round_trip(golden):
    """Under the byte-level vocabularies every byte has a piece, so the
    pieces of the ids spell the text back."""
    g, man = golden
    t = M.Bpe(g["blob_bpe1200"].tobytes())
    for c in man["cases"]:
        if c["vocab"] != "bpe1200" or c["key"] is None:
            continue
        raw = c["text"].encode()
        assert b"".join(t.piece(i) for i in t.encode(raw)) == raw


def test_rejects_bad_blobs(golden):
    g, _ = golden
    good = g["blob_chat"].tobytes()
    for bad in (b"NOPE....", good[:27], good[:-1], b"MTK2" + good[4:],
                good[:4] + struct.pack("<I", 0) + good[8:]):
        with pytest.raises(ValueError):
            M.Bpe(bad)
    # a merge naming an id past the vocabulary
    pieces = [b"a", b"b"]
    with pytest.raises(ValueError):
        M.Bpe(MW.mtk1_blob(pieces, [(0, 1, 2)]))
    with pytest.raises(ValueError):
        M.Bpe(MW.mtk1_blob(pieces, specials=(5,)))


def test_serve_program_command_line(tmp_path):
    assert os.path.exists(M.SERVE_PATH), "motoria_amd/mia-serve is not built"
    r = subprocess.run([M.SERVE_PATH], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
    r = subprocess.run([M.SERVE_PATH, "-m", str(tmp_path / "absent.mia")], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 1 and "open" in r.stderr
    r = subprocess.run([M.SERVE_PATH, "-m", "x.mia", "--bogus", "1"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 2 and "unknown option" in r.stderr
