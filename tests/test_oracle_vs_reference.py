"""The C restatement (oracle/) against the reference's own compiled code
(oracle/_ref, built from the reference sources by `make -C oracle ref`), bit
for bit, on inputs beyond the committed golden vectors. Skipped where the
reference build is absent (the GPU box has no reference sources)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")


def test_quantize_random_rows_bit_equal():
    R = O.ref()
    rng = np.random.default_rng(10)
    for scale in [1e-30, 1e-3, 1.0, 1e6]:
        x = (rng.normal(size=64 * 32) * scale).astype(np.float32)
        x[:32] = 0.0  # a zero block
        want = np.zeros(x.size // 32 * 36, np.uint8)
        R.mia_quantize_row_q8(x.ctypes.data, want.ctypes.data, x.size)
        assert np.array_equal(O.quantize_row_q8(x), want)


@pytest.mark.parametrize("rows,cols,wtype", [(64, 2048, 0), (128, 2048, 0), (768, 2048, 1),
                                             (2048, 768, 1), (3, 32, 1)])
def test_matvec_bit_equal(rows, cols, wtype):
    R = O.ref()
    rng = np.random.default_rng(rows + cols)
    w = (rng.normal(size=rows * cols) * 0.02).astype(np.float32)
    x = rng.normal(size=cols).astype(np.float32)
    if wtype == 1:
        w = np.concatenate([O.quantize_row_q8(w[r * cols:(r + 1) * cols]) for r in range(rows)])
    want = np.zeros(rows, np.float32)
    xq = np.zeros(max(cols // 32, 1) * 36, np.uint8)
    R.mia_matvec_scalar(want.ctypes.data, w.ctypes.data, wtype, x.ctypes.data, xq.ctypes.data,
                        rows, cols)
    assert np.array_equal(O.matvec(w, wtype, x, rows, cols).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("shape,T,seed", [("TINY", 64, 21), ("TINY", 64, 22),
                                          ("QWEN3_30B_A3B", 3, 23)])
def test_layer_bit_equal(shape, T, seed):
    d = O.dims(**getattr(O, shape))
    x = O.synth_x(seed + 100, T, d.dim)
    router = O.synth_router(seed, 0, d)
    norm = (1.0 + 0.1 * np.random.default_rng(seed).normal(size=d.dim)).astype(np.float32)
    blobs = [O.synth_expert_blob(seed, 0, e, d) for e in range(d.n_experts)]
    xo, idx, w, logits, xn = O.moe_layer(d, x, norm, router, blobs, nthreads=4)
    xr, il, ir, wr, lr, xnr = O.ref_moe_layer(d, x, norm, router, blobs)
    assert np.array_equal(idx, ir) and np.array_equal(il, ir)
    for a, b in [(xo, xr), (w, wr), (logits, lr), (xn, xnr)]:
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_tokenizer_random_texts_equal_the_reference():
    """The serve path's tokenizer (host/tokenizer.c) against the reference's
    own (src/tokenizer/bpe.c, through oracle/_ref) on seeded random texts
    built from the characters its rules distinguish: both letter cases,
    digits, space / tab / newline / carriage return, ASCII punctuation,
    apostrophes with contraction letters, two- to four-byte UTF-8 (the C2
    and E2 80 / E3 80 punctuation rows among them), stray continuation
    bytes, special tokens, and multi-byte characters cut by a special token
    or by the end of the text; under the four vocabularies of the golden
    fixtures, and with too small an output for some."""
    import ctypes
    import json
    import os

    import motoria_amd as M

    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "tokenizer.npz"))
    vocabs = sorted(k[5:] for k in g.files if k.startswith("blob_"))
    R = O.ref()
    R.ref_tok_encode.restype = ctypes.c_int
    R.ref_tok_encode.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p,
                                 ctypes.c_void_p, ctypes.c_int]
    atoms = [b"a", b"Z", b"q", b"7", b"0", b" ", b"  ", b"\t", b"\n", b"\r\n", b"\n\n", b"\v",
             b"!", b",", b".", b"(", b"'", b"'s", b"'T", b"'re", b"'VE", b"'ll", b"'d", b"'m",
             b"'x", b"\xc2\xa0", b"\xc2\xbf", b"\xc3\xa9", b"\xe2\x80\x94", b"\xe2\x80\x9c",
             b"\xe3\x80\x82", b"\xe4\xbd\xa0", b"\xe2\x82\xac", b"\xf0\x9f\x98\x80", b"\x80",
             b"\xbf", b"<|im_start|>", b"<|im_end|>", b"<|endoftext|>", b"<think>", b"hello",
             b"Hello", b"world", b"12345", b" the", b"--", b"==>", b"<|im_", b"|>"]
    rng = np.random.default_rng(2024)
    checked = 0
    for v in vocabs:
        blob = g["blob_" + v].tobytes()
        tok = M.Bpe(blob)
        for trial in range(300):
            parts = [atoms[i] for i in rng.integers(0, len(atoms), int(rng.integers(1, 40)))]
            if trial % 7 == 0:  # a multi-byte character cut by a special token or the end
                parts.append(b"\xe4\xbd" if trial % 2 else b"\xf0\x9f\x98")
                if trial % 3 == 0:
                    parts.append(b"<|im_end|>")
            text = b"".join(parts)
            cap = 1 << 14 if trial % 5 else int(rng.integers(1, 12))
            want = np.zeros(cap, np.int32)
            nw = R.ref_tok_encode(blob, len(blob), text, want.ctypes.data, cap)
            got = tok.encode(text, max_ids=cap)
            if nw < 0:
                assert got is None, (v, text)
            else:
                assert got == want[:nw].tolist(), (v, text)
            checked += 1
    assert checked == 300 * len(vocabs)
