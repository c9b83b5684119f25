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
