"""The whole model step on the GPU (mia_gpu_model, include/mia/model_gpu.h).

Embedding, attention with RoPE and the KV cache in HBM, the MoE FFN, final
rmsnorm and output head (src/model/forward.c:199-217 of the reference) over
.mia files written by tests/mia_writer.py:

- the golden models: logits bit-equal to the reference's own mia_model_step
  (tests/golden/model_*.npz, made from oracle/_ref);
- a long context on the tiny model: bit-equal to the oracle's model step at
  every position up to 300;
- two layers of the Qwen3-30B-A3B shape (attention 32/4 heads of 128, MoE
  128 x 768, top-8) with a 1000-token vocabulary: bit-equal to the oracle
  with the exact router (and after forced aborts of the model stack or of
  every attention and decode launch, which rerun per stage); with the certified router (gate weights within
  ~1e-6 relative) the later layers' Q8 requantizations turn that into whole
  quantization steps, ~5e-4 of max|logit| each: max|diff| / max|ref| <= 2e-2,
  and the same top token wherever the reference's top-two margin exceeds
  twice that;
- the full Qwen3-30B-A3B shape (48 layers, vocabulary 151936) generated in
  HBM: the model stack (every layer of a token in one launch), one attention
  and one MoE launch per layer, and the per-stage kernels give the same
  logits bits.
"""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

import motoria_amd as M
import mia_writer as MW

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# The opt-in certified router (MHIP_DECODE_CERTIFIED; the default router is
# exact and every default-flag test here is bit-equal): its gate weights are
# ~1e-6 off, which flips Q8 codes of later layers, so its logits are held to
# the reference's own bar for a Q8_0 model against a float reference,
# 3e-2 of max|ref| (tools/e2e/e2e_test.go:84), with margin.
TOL_CERT = 2e-2


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["model_tiny", "model_mini_qwen"])
def test_model_golden(oracle, tmp_path, name):
    say("test_model_golden", name)
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    spec = json.load(open(os.path.join(GOLDEN, "MANIFEST_model.json")))[name]
    path = str(tmp_path / (name + ".mia"))
    MW.synthetic(oracle, path, spec["cfg"], MW.Q8_0, int(g["seed"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(g["file_sha256"])
    for flags in (M.MHIP_FORCE_EXACT_ROUTER, M.MHIP_EXACT_EXPERTS):
        m = M.GpuModel(path, int(g["max_seq"]), flags=flags)
        try:
            for p, tok in enumerate(g["tokens"].tolist()):
                got = m.step(tok, p)
                assert np.array_equal(bits(got), g["logits_bits"][p]), \
                    "%s flags=%d position %d" % (name, flags, p)
        finally:
            m.close()
        say("  flags=%d: %d positions bit-equal to the reference" % (flags, len(g["tokens"])))


def test_model_tiny_long_context_and_bounds(oracle, tmp_path):
    say("test_model_tiny_long_context_and_bounds")
    path = str(tmp_path / "tiny.mia")
    MW.synthetic(oracle, path, MW.TINY, MW.Q8_0, 21)
    fm = MW.FileModel(oracle, path, MW.TINY)
    max_seq, n = 320, 300
    kc, vc = fm.kv_cache(max_seq)
    toks = np.random.default_rng(5).integers(0, MW.TINY["vocab"], n).tolist()
    m = M.GpuModel(path, max_seq)
    try:
        for p, tok in enumerate(toks):
            want, _ = oracle.model_step(fm.model, kc, vc, max_seq, tok, p, nthreads=4)
            assert np.array_equal(bits(m.step(tok, p)), bits(want)), "position %d" % p
        say("  %d positions bit-equal to the oracle" % n)
        for tok, pos in ((0, max_seq), (0, -1), (MW.TINY["vocab"], 0), (-1, 0)):
            with pytest.raises(RuntimeError, match="outside"):
                m.step(tok, pos)
        # the handle still works after the rejected calls
        want, _ = oracle.model_step(fm.model, kc, vc, max_seq, 7, n, nthreads=4)
        assert np.array_equal(bits(m.step(7, n)), bits(want))
    finally:
        m.close()
    with pytest.raises(RuntimeError, match="max_seq"):
        M.GpuModel(path, 0)
    with pytest.raises(RuntimeError, match="open"):
        M.GpuModel(str(tmp_path / "absent.mia"), 4)
    f32 = str(tmp_path / "f32.mia")
    MW.synthetic(oracle, f32, MW.TINY, MW.F32, 21)
    with pytest.raises(RuntimeError, match="Q8_0"):
        M.GpuModel(f32, 4)


QWEN2 = dict(dim=2048, n_layers=2, n_heads=32, n_kv_heads=4, head_dim=128, vocab=1000,
             n_experts=128, n_active=8, expert_hidden=768, norm_topk=1, rope_theta=1e6,
             norm_eps=1e-6)
QWEN_TOKENS = 24


@pytest.fixture(scope="module")
def qwen_model(oracle, tmp_path_factory):
    """A two-layer Qwen3-30B-A3B-shaped file and the oracle's logits of
    QWEN_TOKENS seeded tokens."""
    path = str(tmp_path_factory.mktemp("qwen") / "qwen2.mia")
    say("write the two-layer Qwen-shaped file")
    MW.synthetic(oracle, path, QWEN2, MW.Q8_0, 31)
    fm = MW.FileModel(oracle, path, QWEN2)
    kc, vc = fm.kv_cache(QWEN_TOKENS)
    toks = np.random.default_rng(8).integers(0, QWEN2["vocab"], QWEN_TOKENS).tolist()
    want = np.stack([oracle.model_step(fm.model, kc, vc, QWEN_TOKENS, t, p, nthreads=8)[0]
                     for p, t in enumerate(toks)])
    del fm
    return path, toks, want


EXACT, PER_LAYER = M.MHIP_FORCE_EXACT_ROUTER, M.MHIP_MODEL_PER_LAYER


# Steps of the model stack (one launch per token: an abort is one launch) and
# of one attention and one MoE launch per layer (MHIP_MODEL_PER_LAYER).
@pytest.mark.parametrize("flags,aborts", [
    (EXACT, 0),
    (EXACT | M.MHIP_DECODE_CHAINS_FIRST, 0),
    (EXACT | M.MHIP_FORCE_SEQ_RMS, 0),
    (EXACT | M.MHIP_DECODE_FORCE_ABORT, 1),
    (EXACT | M.MHIP_ATTN_FORCE_ABORT, 1),
    (EXACT | PER_LAYER, 0),
    (EXACT | PER_LAYER | M.MHIP_DECODE_CHAINS_FIRST, 0),
    (EXACT | PER_LAYER | M.MHIP_FORCE_SEQ_RMS, 0),
    (EXACT | PER_LAYER | M.MHIP_DECODE_FORCE_ABORT, 2),
    (EXACT | PER_LAYER | M.MHIP_ATTN_FORCE_ABORT, 2),
    (EXACT | PER_LAYER | M.MHIP_ATTN_FORCE_ABORT | M.MHIP_DECODE_FORCE_ABORT, 4),
    (M.MHIP_EXACT_EXPERTS, 0),
])
def test_model_qwen_shape_bit_exact(qwen_model, flags, aborts):
    say("test_model_qwen_shape_bit_exact flags=%d" % flags)
    path, toks, want = qwen_model
    m = M.GpuModel(path, QWEN_TOKENS, flags=flags)
    try:
        for p, tok in enumerate(toks):
            got = m.step(tok, p)
            assert m.aborts() == aborts
            assert np.array_equal(bits(got), bits(want[p])), "position %d" % p
    finally:
        m.close()
    say("  %d positions bit-equal to the oracle" % len(toks))


def check_certified(got, want, where):
    err = float(np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)))
    assert err <= TOL_CERT, "%s: rel err %.3g" % (where, err)
    top2 = np.sort(want)[-2:]
    if top2[1] - top2[0] > 2 * TOL_CERT * np.max(np.abs(want)):
        assert int(np.argmax(got)) == int(np.argmax(want)), where
    return err


@pytest.mark.parametrize("flags", [M.MHIP_DECODE_CERTIFIED, M.MHIP_DECODE_CERTIFIED | PER_LAYER])
def test_model_qwen_shape_certified(qwen_model, flags):
    say("test_model_qwen_shape_certified flags=%d" % flags)
    path, toks, want = qwen_model
    m = M.GpuModel(path, QWEN_TOKENS, flags=flags)
    worst = 0.0
    try:
        for p, tok in enumerate(toks):
            got = m.step(tok, p)
            assert m.aborts() == 0
            worst = max(worst, check_certified(got, want[p], "position %d" % p))
    finally:
        m.close()
    say("  worst rel err %.3g over %d positions" % (worst, len(toks)))


QWEN_FULL = dict(dim=2048, n_layers=48, n_heads=32, n_kv_heads=4, head_dim=128, vocab=151936,
                 n_experts=128, n_active=8, expert_hidden=768, norm_topk=1, rope_theta=1e6,
                 norm_eps=1e-6)


def test_model_full_shape_decode_equals_per_stage():
    """48 layers: the model stack (one launch per token), one attention and
    one MoE launch per layer, and the per-stage kernels give the same logits
    bits; the certified router stays within its tolerance."""
    say("test_model_full_shape_decode_equals_per_stage")
    n = 6
    a = M.GpuModel(None, 64, synth=(QWEN_FULL, 5))
    b = M.GpuModel(None, 64, flags=M.MHIP_EXACT_EXPERTS, synth=(QWEN_FULL, 5))
    c = M.GpuModel(None, 64, flags=M.MHIP_DECODE_CERTIFIED, synth=(QWEN_FULL, 5))
    d = M.GpuModel(None, 64, flags=EXACT | PER_LAYER, synth=(QWEN_FULL, 5))
    try:
        toks = np.random.default_rng(3).integers(0, QWEN_FULL["vocab"], n).tolist()
        worst = 0.0
        for p, tok in enumerate(toks):
            la, lb, lc, ld = a.step(tok, p), b.step(tok, p), c.step(tok, p), d.step(tok, p)
            assert a.aborts() == 0 and c.aborts() == 0 and d.aborts() == 0
            assert np.all(np.isfinite(la))
            assert np.array_equal(bits(la), bits(lb)), "position %d" % p
            assert np.array_equal(bits(ld), bits(lb)), "position %d (per layer)" % p
            worst = max(worst, check_certified(lc, lb.astype(np.float64), "position %d" % p))
        say("  %d positions: stack == per-layer == per-stage step; certified worst %.3g" % (n, worst))
    finally:
        a.close()
        b.close()
        c.close()
        d.close()


def test_model_full_shape_one_launch_attention_far_positions():
    """The one-launch attention (in the model stack and per layer) at
    positions past its 512 threads (several scores per thread, a long mix)
    and around its 64 staged cache rows, against the per-stage step;
    positions in between are left empty (zero cache rows), so only the steps
    shown run."""
    say("test_model_full_shape_one_launch_attention_far_positions")
    a = M.GpuModel(None, 2048, synth=(QWEN_FULL, 6))
    b = M.GpuModel(None, 2048, flags=M.MHIP_EXACT_EXPERTS, synth=(QWEN_FULL, 6))
    c = M.GpuModel(None, 2048, flags=EXACT | PER_LAYER, synth=(QWEN_FULL, 6))
    try:
        rng = np.random.default_rng(11)
        for p in (0, 1, 35, 64, 65, 700, 1500, 2047):
            tok = int(rng.integers(0, QWEN_FULL["vocab"]))
            la, lb, lc = a.step(tok, p), b.step(tok, p), c.step(tok, p)
            assert a.aborts() == 0 and c.aborts() == 0
            assert np.all(np.isfinite(la))
            assert np.array_equal(bits(la), bits(lb)), "position %d" % p
            assert np.array_equal(bits(lc), bits(lb)), "position %d (per layer)" % p
        say("  positions 0 .. 2047: model stack == per-layer launches == per-stage")
    finally:
        a.close()
        b.close()
        c.close()


def test_model_full_shape_stack_at_its_longest_context():
    """The model stack's largest context (MHIP_MODEL_STACK_MAX_SEQ positions:
    the last position's 8192 scores fill the dynamic LDS) against the
    per-stage step; one past it the model runs per layer (same bits)."""
    say("test_model_full_shape_stack_at_its_longest_context")
    n = M.MHIP_MODEL_STACK_MAX_SEQ
    a = M.GpuModel(None, n, synth=(QWEN_FULL, 8))
    b = M.GpuModel(None, n, flags=M.MHIP_EXACT_EXPERTS, synth=(QWEN_FULL, 8))
    c = M.GpuModel(None, n + 1, synth=(QWEN_FULL, 8))
    try:
        rng = np.random.default_rng(12)
        for p in (0, 33, n // 2, n - 1):
            tok = int(rng.integers(0, QWEN_FULL["vocab"]))
            la, lb, lc = a.step(tok, p), b.step(tok, p), c.step(tok, p)
            assert a.aborts() == 0 and c.aborts() == 0
            assert np.all(np.isfinite(la))
            assert np.array_equal(bits(la), bits(lb)), "position %d" % p
            assert np.array_equal(bits(lc), bits(lb)), "position %d (max_seq %d)" % (p, n + 1)
        say("  positions 0, 33, %d, %d: stack == per-stage == per-layer" % (n // 2, n - 1))
    finally:
        a.close()
        b.close()
        c.close()


def test_model_long_context_attention_paths_agree(oracle, tmp_path):
    """The per-head attention kernel keeps the scores in LDS; a context too
    long for that runs the separate score and mix kernels. Both give the
    same logits (the mini Qwen shape, head_dim 128, 40 positions, with a
    4096-position and a 40000-position cache)."""
    say("test_model_long_context_attention_paths_agree")
    spec = json.load(open(os.path.join(GOLDEN, "MANIFEST_model.json")))["model_mini_qwen"]
    path = str(tmp_path / "mini.mia")
    MW.synthetic(oracle, path, spec["cfg"], MW.Q8_0, 9)
    toks = np.random.default_rng(4).integers(0, spec["cfg"]["vocab"], 40).tolist()
    a = M.GpuModel(path, 4096)
    b = M.GpuModel(path, 40000)
    try:
        for p, tok in enumerate(toks):
            assert np.array_equal(bits(a.step(tok, p)), bits(b.step(tok, p))), "position %d" % p
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("name", ["model_tiny", "model_mini_qwen"])
def test_model_prefill_equals_feeds_golden(oracle, tmp_path, name):
    """mia_gpu_model_prefill of the first k tokens, then steps: the logits are
    the reference's own (the golden files) at every later position, for k
    across the 64-token batch size."""
    say("test_model_prefill_equals_feeds_golden", name)
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    spec = json.load(open(os.path.join(GOLDEN, "MANIFEST_model.json")))[name]
    path = str(tmp_path / (name + ".mia"))
    MW.synthetic(oracle, path, spec["cfg"], MW.Q8_0, int(g["seed"]))
    toks = g["tokens"].tolist()
    n = len(toks)
    m = M.GpuModel(path, int(g["max_seq"]))
    try:
        for k in sorted({1, n // 2, n - 1}):
            m.prefill(toks[:k], 0)
            for p in range(k, n):
                got = m.step(toks[p], p)
                assert np.array_equal(bits(got), g["logits_bits"][p]), \
                    "%s prefill %d, position %d" % (name, k, p)
        say("  prefill of 1, %d, %d tokens then steps: bit-equal to the reference" % (n // 2, n - 1))
        with pytest.raises(RuntimeError, match="outside"):
            m.prefill([0, 1], int(g["max_seq"]) - 1)
    finally:
        m.close()


@pytest.mark.parametrize("n", [70, 300, 1100])
def test_model_full_shape_prefill_equals_feeds(n):
    """48 layers at the Qwen3-30B-A3B shape: an n-token prompt through
    mia_gpu_model_prefill, then steps, gives the logits bits of n feeds and
    the same steps. 70 tokens: one batch, its MoE on the vector kernels (560
    assignments); 300: one batch on the matrix-core kernels (2400); 1100: two
    batches of 550, each nine 64-token row chunks (the last partial)."""
    say("test_model_full_shape_prefill_equals_feeds n=%d" % n)
    a = M.GpuModel(None, 1200, synth=(QWEN_FULL, 9))
    b = M.GpuModel(None, 1200, synth=(QWEN_FULL, 9))
    try:
        toks = np.random.default_rng(13).integers(0, QWEN_FULL["vocab"], n + 3).tolist()
        a.prefill(toks[:n], 0)
        for p in range(n):
            b.feed(toks[p], p)
        for p in range(n, n + 3):
            la, lb = a.step(toks[p], p), b.step(toks[p], p)
            assert np.all(np.isfinite(la))
            assert np.array_equal(bits(la), bits(lb)), "position %d" % p
        say("  %d-token prefill + 3 steps == %d feeds + 3 steps (bits)" % (n, n))
    finally:
        a.close()
        b.close()


def test_model_full_shape_prefill_far_positions():
    """A prompt batch whose context is too long for its scores in LDS (the
    scores in device memory, 64 tokens per pass: 70 tokens at positions
    4300 .. 4369), against feeds; the positions before are left empty (zero
    cache rows) on both handles."""
    say("test_model_full_shape_prefill_far_positions")
    a = M.GpuModel(None, 4400, synth=(QWEN_FULL, 10))
    b = M.GpuModel(None, 4400, synth=(QWEN_FULL, 10))
    try:
        toks = np.random.default_rng(14).integers(0, QWEN_FULL["vocab"], 75).tolist()
        a.prefill(toks[:3], 0)
        a.prefill(toks[3:73], 4300)
        for p in range(3):
            b.feed(toks[p], p)
        for p in range(70):
            b.feed(toks[3 + p], 4300 + p)
        for p, tok in ((4370, toks[73]), (4371, toks[74])):
            la, lb = a.step(tok, p), b.step(tok, p)
            assert np.all(np.isfinite(la))
            assert np.array_equal(bits(la), bits(lb)), "position %d" % p
        say("  prefill at 4300 .. 4369 + 2 steps == feeds + 2 steps (bits)")
    finally:
        a.close()
        b.close()
