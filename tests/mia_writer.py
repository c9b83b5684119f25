"""Writes .mia model files for the tests.

The layout is the reference converter's (tools/internal/mia/format.go):
a 112-byte little-endian header in a 16 KiB region, the dense tensors from
offset 16384 in NewLayout's order (:129-165; matrices in the file's weight
type, vectors and routers fp32, each tensor 64-byte aligned), then one
16 KiB-aligned blob per (layer, expert) holding gate, up and down at the
blob offsets of :160-163, then the tokenizer (WriteFile, :200-263). The
tensors are synthetic: the caller supplies them.
"""
import struct

import numpy as np

HEADER_REGION = 16384
TENSOR_ALIGN = 64
EXPERT_ALIGN = 16384
F32, Q8_0 = 0, 1
HEADER = struct.Struct("<4s12I2fI6Q")
assert HEADER.size == 112

# The reference's tiny e2e model (tools/e2e/e2e_test.go:23-29).
TINY = dict(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, vocab=96,
            n_experts=8, n_active=2, expert_hidden=32, norm_topk=1, rope_theta=1e6,
            norm_eps=1e-6)


def align(n, a):
    return (n + a - 1) // a * a


def mat_bytes(wtype, rows, cols):
    return rows * (cols // 32) * 36 if wtype == Q8_0 else rows * cols * 4


def layout(cfg, wtype):
    """Dense entries [(name, rows, cols, quantized, offset)], dense size,
    blob offsets (up, down) and blob size."""
    d, hd, V = cfg["dim"], cfg["head_dim"], cfg["vocab"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    entries, off = [], 0

    def add(name, rows, cols, quant):
        nonlocal off
        entries.append((name, rows, cols, quant, off))
        nbytes = mat_bytes(wtype, rows, cols) if quant else rows * cols * 4
        off = align(off + nbytes, TENSOR_ALIGN)

    add("token_embd", V, d, True)
    for i in range(cfg["n_layers"]):
        p = "blk.%d." % i
        add(p + "attn_norm", 1, d, False)
        add(p + "wq", qd, d, True)
        add(p + "wk", kvd, d, True)
        add(p + "wv", kvd, d, True)
        add(p + "wo", d, qd, True)
        add(p + "q_norm", 1, hd, False)
        add(p + "k_norm", 1, hd, False)
        add(p + "ffn_norm", 1, d, False)
        add(p + "router", cfg["n_experts"], d, False)
    add("output_norm", 1, d, False)
    add("output", V, d, True)
    up = align(mat_bytes(wtype, cfg["expert_hidden"], d), TENSOR_ALIGN)
    down = up + align(mat_bytes(wtype, cfg["expert_hidden"], d), TENSOR_ALIGN)
    blob = align(down + mat_bytes(wtype, d, cfg["expert_hidden"]), EXPERT_ALIGN)
    return entries, off, up, down, blob


def write(path, cfg, wtype, dense, expert_blob, tokenizer=b""):
    """dense(name, rows, cols) -> float32 values (row-major); expert_blob(l,
    e) -> the blob's bytes (gate at 0, up and down at the layout's offsets).
    Quantized matrices of a Q8_0 file are encoded with encode_q8 (the
    caller's quantizer). Returns the layout."""
    entries, dense_size, up, down, blob = layout(cfg, wtype)
    experts_offset = align(HEADER_REGION + dense_size, EXPERT_ALIGN)
    n_blobs = cfg["n_layers"] * cfg["n_experts"]
    tok_offset = experts_offset + n_blobs * blob
    hdr = HEADER.pack(b"MIA1", 1, wtype, cfg["dim"], cfg["n_layers"], cfg["n_heads"],
                      cfg["n_kv_heads"], cfg["head_dim"], cfg["vocab"], cfg["n_experts"],
                      cfg["n_active"], cfg["expert_hidden"], cfg["norm_topk"],
                      cfg["rope_theta"], cfg["norm_eps"], 0, HEADER_REGION, dense_size,
                      experts_offset, blob, tok_offset, len(tokenizer))
    with open(path, "wb") as f:
        f.write(hdr)
        for name, rows, cols, quant, off in entries:
            x = np.ascontiguousarray(dense(name, rows, cols), dtype=np.float32)
            assert x.size == rows * cols, name
            f.seek(HEADER_REGION + off)
            f.write(encode_q8(x) if quant and wtype == Q8_0 else x.tobytes())
        for l in range(cfg["n_layers"]):
            for e in range(cfg["n_experts"]):
                b = bytes(expert_blob(l, e))
                assert len(b) == blob, (len(b), blob)
                f.seek(experts_offset + (l * cfg["n_experts"] + e) * blob)
                f.write(b)
        f.seek(tok_offset)
        f.write(tokenizer)
    return dict(entries={e[0]: e for e in entries}, dense_size=dense_size, off_up=up,
                off_down=down, blob=blob, experts_offset=experts_offset, tok_offset=tok_offset)


encode_q8 = None  # set by the caller: float32 values -> Q8_0 bytes (per 32-value block)


def synthetic(O, path, cfg, wtype=Q8_0, seed=7, tokenizer=b"tok"):
    """A synthetic model file: dense tensors ~ N(0, 0.02) from numpy's
    seeded generator (norms 1 + 0.1 N(0, 1); routers N(0, 0.16) so routing is
    decisive), Q8_0 matrices quantized with the oracle's quantizer, experts
    from the synthetic generator (Q8_0 files) or fp32 normals (F32 files).
    O is the oracle module. Returns the layout of `write`."""
    global encode_q8
    encode_q8 = O.quantize_row_q8
    rng = np.random.default_rng(seed)
    d = O.dims(dim=cfg["dim"], n_experts=cfg["n_experts"], n_active=cfg["n_active"],
               expert_hidden=cfg["expert_hidden"], norm_topk=cfg["norm_topk"],
               norm_eps=cfg["norm_eps"])

    def dense(name, rows, cols):
        if "norm" in name:
            return 1.0 + 0.1 * rng.standard_normal(rows * cols)
        if name.endswith("router"):
            return 0.4 * rng.standard_normal(rows * cols)
        return 0.02 * rng.standard_normal(rows * cols)

    _, _, up, down, blob = layout(cfg, wtype)

    def expert(l, e):
        if wtype == Q8_0:
            return O.synth_expert_blob(seed + l, l, e, d)
        b = np.zeros(blob, np.uint8)
        eh, dim = cfg["expert_hidden"], cfg["dim"]
        for off, n in ((0, eh * dim), (up, eh * dim), (down, dim * eh)):
            b[off:off + 4 * n] = (0.02 * rng.standard_normal(n)).astype(np.float32).view(np.uint8)
        return b

    return write(path, cfg, wtype, dense, expert, tokenizer=tokenizer)


# A model with the attention shape of Qwen3-30B-A3B (dim 2048, 32 query and 4
# key/value heads of 128) and a smaller MoE and vocabulary, for model-step
# tests that run on the CPU.
MINI_QWEN = dict(dim=2048, n_layers=2, n_heads=32, n_kv_heads=4, head_dim=128, vocab=64,
                 n_experts=16, n_active=4, expert_hidden=768, norm_topk=1, rope_theta=1e6,
                 norm_eps=1e-6)


def read_dense(path, lay, name):
    """A dense fp32 tensor back from the file (vectors and routers)."""
    _, rows, cols, quant, off = lay["entries"][name]
    assert not quant
    with open(path, "rb") as f:
        f.seek(HEADER_REGION + off)
        return np.frombuffer(f.read(rows * cols * 4), dtype=np.float32).reshape(rows, cols)


def read_blob(path, lay, cfg, layer, expert):
    with open(path, "rb") as f:
        f.seek(lay["experts_offset"] + (layer * cfg["n_experts"] + expert) * lay["blob"])
        return np.frombuffer(f.read(lay["blob"]), dtype=np.uint8)


class FileModel:
    """An oracle.Model over the bytes of a .mia file written by `write`
    (Q8_0), with the pointer arrays it needs kept alive."""

    def __init__(self, O, path, cfg):
        import ctypes
        self.data = np.fromfile(path, dtype=np.uint8)
        entries, _, _, _, blob = layout(cfg, Q8_0)
        entries = {e[0]: e for e in entries}
        base = self.data.ctypes.data
        experts_offset = align(HEADER_REGION + layout(cfg, Q8_0)[1], EXPERT_ALIGN)
        L, E = cfg["n_layers"], cfg["n_experts"]

        def ptr(name):
            return base + HEADER_REGION + entries[name][4]

        def arr(names):
            a = (ctypes.c_void_p * len(names))(*[ptr(n) for n in names])
            self.keep.append(a)
            return ctypes.cast(a, ctypes.c_void_p)

        self.keep = []
        m = O.Model()
        m.moe = O.dims(dim=cfg["dim"], n_experts=E, n_active=cfg["n_active"],
                       expert_hidden=cfg["expert_hidden"], norm_topk=cfg["norm_topk"],
                       norm_eps=cfg["norm_eps"])
        m.n_layers, m.n_heads, m.n_kv_heads = L, cfg["n_heads"], cfg["n_kv_heads"]
        m.head_dim, m.vocab, m.wtype, m.rope_theta = (cfg["head_dim"], cfg["vocab"], Q8_0,
                                                      cfg["rope_theta"])
        m.token_embd, m.output, m.output_norm = ptr("token_embd"), ptr("output"), ptr("output_norm")
        for field, suffix in (("attn_norm", "attn_norm"), ("q_norm", "q_norm"), ("k_norm", "k_norm"),
                              ("ffn_norm", "ffn_norm"), ("router", "router"), ("wq", "wq"),
                              ("wk", "wk"), ("wv", "wv"), ("wo", "wo")):
            setattr(m, field, arr(["blk.%d.%s" % (l, suffix) for l in range(L)]))
        blobs = (ctypes.c_void_p * (L * E))(
            *[base + experts_offset + i * blob for i in range(L * E)])
        self.keep.append(blobs)
        m.blobs = ctypes.cast(blobs, ctypes.c_void_p)
        self.model = m
        self.cfg = cfg

    def kv_cache(self, max_seq):
        c = self.cfg
        n = c["n_layers"] * max_seq * c["n_kv_heads"] * c["head_dim"]
        return np.zeros(n, np.float32), np.zeros(n, np.float32)


# ---- MTK1 tokenizer blobs (the reader's format, src/tokenizer/bpe.c:35-95) --------

NO_ID = 0xFFFFFFFF


def mtk1_blob(pieces, merges=(), specials=(), eos=None, im_start=None, im_end=None):
    """pieces: byte strings (id = index); merges: (a, b, result) in rank
    order; specials: ids matched literally before pre-tokenization; eos /
    im_start / im_end: ids or None."""
    opt = lambda v: NO_ID if v is None else v  # noqa: E731
    out = [b"MTK1", struct.pack("<6I", len(pieces), len(merges), len(specials), opt(eos),
                                opt(im_start), opt(im_end))]
    for p in pieces:
        out.append(struct.pack("<H", len(p)) + p)
    for a, b, r in merges:
        out.append(struct.pack("<3I", a, b, r))
    for s in specials:
        out.append(struct.pack("<I", s))
    return b"".join(out)


def chat_tokenizer():
    """The reference's serve test vocabulary (tools/e2e/serve_test.go:16-33):
    ids 0..91 are '!'..'|', 92 space, 93 newline, 94 <|im_start|>,
    95 <|im_end|>; no merges."""
    pieces = [bytes([33 + i]) for i in range(92)] + [b" ", b"\n", b"<|im_start|>",
                                                     b"<|im_end|>"]
    return mtk1_blob(pieces, specials=(94, 95), im_start=94, im_end=95)


def trained_tokenizer(corpus, n_merges, seed=0):
    """A byte-level BPE vocabulary: the 256 bytes in a seeded order, then
    n_merges merges trained greedily on `corpus` (most frequent adjacent
    pair, ties to the smaller pair), plus three specials; a duplicate merge
    pair and a duplicate single-byte piece exercise the reader's
    first-wins rules."""
    import random
    rnd = random.Random(seed)
    order = list(range(256))
    rnd.shuffle(order)
    pieces = [bytes([b]) for b in order]
    byte_id = {b: i for i, b in enumerate(order)}
    words = [[byte_id[c] for c in w.encode()] for w in corpus.split(" ") if w]
    merges = []
    for _ in range(n_merges):
        counts = {}
        for w in words:
            for x, y in zip(w, w[1:]):
                counts[(x, y)] = counts.get((x, y), 0) + 1
        if not counts:
            break
        pair = min(counts, key=lambda k: (-counts[k], k))
        new = len(pieces)
        pieces.append(pieces[pair[0]] + pieces[pair[1]])
        merges.append((pair[0], pair[1], new))
        for w in words:
            i = 0
            while i + 1 < len(w):
                if (w[i], w[i + 1]) == pair:
                    w[i:i + 2] = [new]
                i += 1
    merges.append((merges[0][0], merges[0][1], merges[-1][2]))  # duplicate pair: rank 0 wins
    pieces.append(pieces[0])                                     # duplicate byte: first id wins
    base = len(pieces)
    pieces += [b"<|endoftext|>", b"<|im_start|>", b"<|im_end|>"]
    return mtk1_blob(pieces, merges, specials=(base, base + 1, base + 2), eos=base,
                     im_start=base + 1, im_end=base + 2), len(pieces)
