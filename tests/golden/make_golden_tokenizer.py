"""Writes tests/golden/tokenizer.npz: token ids the reference's own
tokenizer (src/tokenizer/bpe.c, through oracle/_ref) gives for texts under
four MTK1 vocabularies, and the reference's chat-template text
(src/model/runtime.c:84-95) for every flag combination.

Run in the container that holds the reference sources, after
`make -C oracle ref`:

    python tests/golden/make_golden_tokenizer.py

Vocabularies (tests/mia_writer.py): the reference's unit-test blob
(tests/test_tokenizer.c:24-39), the serve test's chat vocabulary
(tools/e2e/serve_test.go:16-33), and two byte-level BPE vocabularies with
300 and 1200 merges trained on the corpus below.
"""
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle as O  # noqa: E402
import mia_writer as MW  # noqa: E402

CORPUS = (
    "The quick brown fox jumps over the lazy dog. It's the fox's den; they're "
    "sure we'll see it'd go. Numbers 12345 and 3.14159 or 2024-12-02! "
    "def main(argv):\n    return argv[0] + 'x' * 42  # comment\n"
    "Grüße aus München, señor niño. 中文字符测试 한국어 テスト 🙂🚀 "
    "<b>tags</b> & entities &amp; \"quotes\" (parens) [brackets] {braces} "
    "spaces    and\ttabs\r\nCRLF lines\n\n\nblank lines ¿qué? ¡sí! «guillemets» "
    "—dashes— and… ellipses “smart quotes” ‘single’ "
) * 3

TEXTS = [
    "", "a", "abc abc", "ba", "abc<|im_end|>abc", "abc!abc", "abc abc!<|im_end|>",
    "Hello world", "Hello  world", "Hello   world\n", " leading", "trailing ",
    "it's they're we'll I'd you've he's 'tis", "'S 'T 'RE 'Ll", "don't'",
    "x = 123456789 + 3.14", "2024-12-02T10:00", "a1b2c3", "   ", "\n\n\n", "\r\n", "\t\tx",
    "  \n  x", "!!!???", " !!! ", "...\n", "(x)\n\n", "Grüße, señor", "中文字符测试",
    "한국어 テスト", "🙂🚀 emoji", "¿qué? ¡sí!", "«a» —b— c… “d” ‘e’", " nbsp thin",
    "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n",
    "<|im_start|><|im_end|><|endoftext|>", "<|im_start|", "<|im_end|>x<|im_end|>",
    "def f(a, b):\n    return a*b  # mult\n", "<b>tags</b> &amp;",
    "The quick brown fox jumps over the lazy dog.", CORPUS[:400],
    "aaaaaaaaaaaaaaaa", "ababababab", "theeeee thethe the the",
]


def ref_encode(blob, text, max_ids=4096):
    R = O.ref()
    R.ref_tok_encode.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p,
                                 ctypes.c_void_p, ctypes.c_int]
    out = np.zeros(max_ids, np.int32)
    n = R.ref_tok_encode(blob, len(blob), text.encode(), out.ctypes.data, max_ids)
    return out[:n].tolist() if n >= 0 else n


def unit_blob():
    pieces = [b"a", b"b", b"c", b" ", b"ab", b"abc", b" abc", b"<|im_end|>", b"!", b"x"]
    return MW.mtk1_blob(pieces, [(0, 1, 4), (4, 2, 5), (3, 5, 6)], specials=(7,), im_end=7)


def vocabularies():
    b300, _ = MW.trained_tokenizer(CORPUS, 300, seed=1)
    b1200, _ = MW.trained_tokenizer(CORPUS, 1200, seed=2)
    return {"unit": unit_blob(), "chat": MW.chat_tokenizer(), "bpe300": b300, "bpe1200": b1200}


def main():
    arrays, cases = {}, []
    for vname, blob in vocabularies().items():
        arrays["blob_" + vname] = np.frombuffer(blob, np.uint8)
        for i, text in enumerate(TEXTS):
            ids = ref_encode(blob, text)
            assert ids != -2, vname
            key = "%s_%d" % (vname, i)
            arrays["ids_" + key] = np.array(ids if ids != -1 else [], np.int32)
            cases.append(dict(vocab=vname, text=text, key=key, overflow=ids == -1))
        # overflow: room for fewer ids than the text needs
        full = ref_encode(blob, TEXTS[-4])
        short = ref_encode(blob, TEXTS[-4], max_ids=max(len(full) - 1, 0))
        cases.append(dict(vocab=vname, text=TEXTS[-4], key=None, max=len(full) - 1,
                          overflow=short == -1))
    R = O.ref()
    R.mia_chat_turn.restype = ctypes.c_void_p
    R.mia_chat_turn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
    libc = ctypes.CDLL(None)
    chat = []
    for user in ("hi", "", "multi\nline <b>"):
        for think in (0, 1):
            for cont in (0, 1):
                p = R.mia_chat_turn(user.encode(), think, cont)
                chat.append(dict(user=user, think=think, continuing=cont,
                                 text=ctypes.string_at(p).decode()))
                libc.free(ctypes.c_void_p(p))
    arrays["manifest"] = np.array(json.dumps(dict(cases=cases, chat=chat)))
    np.savez(os.path.join(HERE, "tokenizer.npz"), **arrays)
    print(len(cases), "encodings,", len(chat), "chat texts")


if __name__ == "__main__":
    main()
