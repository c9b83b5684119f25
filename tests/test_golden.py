"""The CPU oracle reproduces, bit for bit, the golden vectors written by the
reference's own compiled code (tests/golden/make_golden.py). These pin the
oracle wherever the reference sources are absent (e.g. the GPU box)."""
import os

import numpy as np
import pytest

from helpers import bits, sha_bytes, xorshift_uniform

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def test_quantize_golden(oracle):
    g = load("quant")
    x = (xorshift_uniform(4096) * np.float32(3.0)).astype(np.float32)
    assert np.array_equal(sha_bytes(x), g["x_sha"])
    assert np.array_equal(oracle.quantize_row_q8(x), g["q"])


@pytest.mark.parametrize("rows,cols", [(7, 32), (1024, 512)])
def test_matvec_f32_golden(oracle, rows, cols):
    g = load("matvec_f32_%dx%d" % (rows, cols))
    u = xorshift_uniform(2048 * 768 + 768)
    w = u[: rows * cols].copy()
    x = u[rows * cols: rows * cols + cols].copy()
    assert np.array_equal(sha_bytes(w), g["w_sha"]) and np.array_equal(sha_bytes(x), g["x_sha"])
    assert np.array_equal(bits(oracle.matvec(w, 0, x, rows, cols)), bits(g["out"]))


@pytest.mark.parametrize("rows,cols", [(5, 64), (2048, 768)])
def test_matvec_q8_golden(oracle, rows, cols):
    g = load("matvec_q8_%dx%d" % (rows, cols))
    u = xorshift_uniform(2048 * 768 + 768)
    w = u[: rows * cols].copy()
    x = u[rows * cols: rows * cols + cols].copy()
    wq = np.concatenate([oracle.quantize_row_q8(w[r * cols:(r + 1) * cols]) for r in range(rows)])
    assert np.array_equal(sha_bytes(wq), g["w_sha"]) and np.array_equal(sha_bytes(x), g["x_sha"])
    assert np.array_equal(bits(oracle.matvec(wq, 1, x, rows, cols)), bits(g["out"]))


@pytest.mark.parametrize("name,shape_key,wseed,xseed,T", [
    ("layer_tiny", "TINY", 5, 11, 32),
    ("layer_qwen_decode", "QWEN3_30B_A3B", 42, 43, 4),
])
def test_layer_golden(oracle, name, shape_key, wseed, xseed, T):
    g = load(name)
    d = oracle.dims(**getattr(oracle, shape_key))
    x = oracle.synth_x(xseed, T, d.dim)
    assert np.array_equal(sha_bytes(x), g["x_in_sha"])
    blobs = [None] * d.n_experts
    for k, e in enumerate(g["used"].tolist()):
        blobs[e] = oracle.synth_expert_blob(wseed, 0, e, d)
        assert np.array_equal(sha_bytes(blobs[e]), g["blob_sha"][k]), "expert %d bytes" % e
    router = oracle.synth_router(wseed, 0, d)
    norm = np.ones(d.dim, np.float32)
    xo, idx, w, logits, xn = oracle.moe_layer(d, x, norm, router, blobs)
    assert np.array_equal(idx, g["idx"])
    for got, key in [(xn, "xn"), (logits, "logits"), (w, "w"), (xo, "x_out")]:
        assert np.array_equal(bits(got), bits(g[key])), key
