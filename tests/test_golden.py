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


# ---- token sampler (tests/golden/make_golden_sampler.py) --------------------------

def sampler_cases(oracle):
    """(name, logits, temperature, top_p, seed, draws, tokens) of every case
    in tests/golden/sampler.npz."""
    import json
    g = load("sampler")
    out = []
    for c in json.loads(str(g["manifest"])):
        if "logit_seed" in c:
            lg = (np.float32(c["scale"]) * oracle.synth_x(c["logit_seed"], 1, c["n"])[0])
            lg = lg.astype(np.float32)
        else:
            lg = g["logits_" + c["name"]]
        out.append((c["name"], lg, c["t"], c["p"], c["seed"], c["draws"],
                    g["tokens_" + c["name"]].tolist()))
    return out


def test_sampler_golden(oracle):
    """orc_sample picks the reference's own tokens (src/tokenizer/sampler.c:
    33-66), including the reference's unit tests (tests/test_sampler.c:4-32:
    greedy argmax, a tiny top_p keeps only the best, two equal logits both
    drawn > 850 times in 2000)."""
    for name, lg, t, p, seed, draws, want in sampler_cases(oracle):
        assert oracle.sample(lg, t, p, seed, draws) == want, name
    cases = {c[0]: c for c in sampler_cases(oracle)}
    assert cases["greedy_argmax"][6] == [1]
    assert set(cases["tiny_top_p"][6]) == {1}
    pair = cases["equal_pair"][6]
    assert pair.count(0) > 850 and pair.count(1) > 850


def test_sampler_rand01_is_xorshift64star(oracle):
    """The draw is the top 24 bits of xorshift64* (Vigna's published
    generator: x ^= x >> 12, x ^= x << 25, x ^= x >> 27, output x times
    2685821657736338717 mod 2^64), computed here with Python integers."""
    import ctypes
    s = oracle.Sampler()
    oracle.lib().orc_sampler_init(ctypes.byref(s), 1.0, 1.0, 10, 12345)
    x, M = 12345, (1 << 64) - 1
    for _ in range(1000):
        x ^= x >> 12
        x ^= (x << 25) & M
        x ^= x >> 27
        want = ((x * 2685821657736338717) & M) >> 40
        assert oracle.lib().orc_sampler_rand01(ctypes.byref(s)) == np.float32(want / 16777216.0)
    oracle.lib().orc_sampler_init(ctypes.byref(s), 1.0, 1.0, 10, 0)
    assert s.rng == 0x2545F4914F6CDD1D


def test_sampler_greedy_brute_force(oracle):
    """Greedy is the first maximum; NaN never wins except at index 0 (the
    reference's strict comparison, sampler.c:34-37), checked against numpy."""
    rng = np.random.default_rng(4)
    for n in (1, 2, 7, 100, 4096):
        for _ in range(20):
            lg = np.round(rng.standard_normal(n) * 3).astype(np.float32)
            if n > 3 and rng.random() < 0.5:
                lg[rng.integers(1, n, 3)] = np.nan
            want = int(np.nanargmax(lg)) if not np.all(np.isnan(lg[1:])) or n == 1 else 0
            if np.isnan(lg[0]):
                want = 0
            assert oracle.sample(lg, 0.0, 1.0, 1, 1) == [want]
