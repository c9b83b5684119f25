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


# ---- whole-model step (tests/golden/make_golden_model.py) -------------------------

@pytest.mark.parametrize("name", ["model_tiny", "model_mini_qwen"])
def test_model_step_golden(oracle, tmp_path, name):
    """orc_model_step (embedding, attention with RoPE and the KV cache, MoE,
    output head) bit-equal to the reference's own mia_model_step logits, on
    the .mia file the test writer regenerates from the fixture's seed."""
    import hashlib
    import json
    import mia_writer as MW

    g = load(name)
    spec = json.load(open(os.path.join(GOLDEN, "MANIFEST_model.json")))[name]
    path = str(tmp_path / (name + ".mia"))
    MW.synthetic(oracle, path, spec["cfg"], MW.Q8_0, int(g["seed"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(g["file_sha256"]), \
        "the writer no longer reproduces the fixture's file"
    fm = MW.FileModel(oracle, path, spec["cfg"])
    max_seq = int(g["max_seq"])
    kc, vc = fm.kv_cache(max_seq)
    want = g["logits_bits"]
    for p, tok in enumerate(g["tokens"].tolist()):
        lg, _ = oracle.model_step(fm.model, kc, vc, max_seq, tok, p, nthreads=4)
        assert np.array_equal(lg.view(np.uint32), want[p]), "position %d" % p


def test_rope_known_answers(oracle):
    """forward.c:84-93: position 0 is the identity; otherwise element i and
    i + hd/2 rotate by pos * theta^(-2i/hd) (closed form in double, to one
    float rounding), which keeps each pair's norm."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128).astype(np.float32)
    assert np.array_equal(oracle.rope_row(x, 0, 1e6).view(np.uint32), x.view(np.uint32))
    for pos in (1, 7, 1000):
        y = oracle.rope_row(x, pos, 1e6)
        i = np.arange(64)
        a = pos * np.power(1e6, -2.0 * i / 128)
        x0, x1 = x[:64].astype(np.float64), x[64:].astype(np.float64)
        want0 = (x0 * np.cos(a) - x1 * np.sin(a)).astype(np.float32)
        want1 = (x0 * np.sin(a) + x1 * np.cos(a)).astype(np.float32)
        ulp = np.spacing(np.abs(np.concatenate([want0, want1])))
        assert np.all(np.abs(y - np.concatenate([want0, want1])) <= ulp)
        assert np.allclose(y[:64] ** 2 + y[64:] ** 2, x[:64] ** 2 + x[64:] ** 2, rtol=1e-5)
