"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Integer and index results (expert indices, dispatch order, Q8 codes) must be
bit-equal. The fp32 results are required bit-equal too, on the vector path
(small batches, or MHIP_EXACT_EXPERTS) and on the matrix-core path (large
batches): the kernels keep the reference's rounding order, so any difference
is a defect. With MHIP_FAST_DOWN (the matrix-core down terms as fused
multiply-adds, an option) routing stays bit-equal and the layer output must
be within the reference's e2e tolerance, max|diff| / max|ref| <= 1e-3
(tools/e2e/e2e_test.go:101-107), for both the update x_out - x_in and x_out.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

import motoria_amd as M
from motoria_amd import workloads as W

pytestmark = pytest.mark.gpu

NTHREADS = min(16, os.cpu_count() or 1)
TOL = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rel_err(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def assert_bits(a, b, what):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.float32:
        same = bits(a) == bits(b)
        if not same.all():
            n = int((~same).sum())
            raise AssertionError("%s: %d of %d values differ (rel err %.3e)"
                                 % (what, n, a.size, rel_err(a, b)))
    else:
        assert np.array_equal(a, b), what


def oracle_layer(O, moe, d, layer, x, router, bias=None, need=None):
    """Run the oracle on experts read back from the HBM table."""
    blobs = [None] * d.n_experts
    experts = range(d.n_experts) if need is None else sorted(set(need))
    for e in experts:
        blobs[e] = moe.read_expert(layer, e)
    norm = np.ones(d.dim, np.float32)
    return O.moe_layer(d, x, norm, router, blobs, bias=bias, nthreads=NTHREADS)


@pytest.fixture(scope="module")
def qwen_moe():
    say("open qwen handle: 2 layers, max_tokens 2048")
    moe = M.Moe(n_layers=2, max_tokens=2048, device=0, **W.SHAPE)
    moe.synth(W.WEIGHT_SEED)
    moe.sync()
    yield moe
    moe.close()


# ---- tensor ops ------------------------------------------------------------------

def _xorshift_uniform(n, state=0x9E3779B9):
    """The reference tests' deterministic generator (tests/check.h:37-44)."""
    out = np.zeros(n, dtype=np.float32)
    g = state
    for i in range(n):
        g ^= (g << 13) & 0xFFFFFFFF
        g ^= g >> 17
        g ^= (g << 5) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(g & 0xFFFFFF) / np.float32(0x1000000) * np.float32(2.0)
                            - np.float32(1.0))
    return out


def test_quantize_known_answers(oracle):
    say("test_quantize_known_answers")
    L = M.lib()
    x = np.zeros(32, np.float32)
    x[3], x[7] = -2.0, 1.0
    y = np.zeros(36, np.uint8)
    L.mia_quantize_row_q8(x.ctypes.data, y.ctypes.data, 32)
    q = y[4:].view(np.int8)
    assert q[3] == -127 and q[7] == 64  # tests/test_quant.c:33-41
    z = np.zeros(32, np.float32)
    L.mia_quantize_row_q8(z.ctypes.data, y.ctypes.data, 32)
    assert y[:4].view(np.float32)[0] == 0.0 and not y[4:].any()


def test_quantize_and_matvec_bit_exact(oracle):
    say("test_quantize_and_matvec_bit_exact")
    L = M.lib()
    u = _xorshift_uniform(2048 * 768 + 4096)
    for rows, cols in [(5, 64), (2048, 768), (7, 32), (1024, 512)]:
        w = (u[: rows * cols] * 3.0).astype(np.float32)
        x = u[rows * cols: rows * cols + cols].copy()
        # Q8 rows
        wq = np.concatenate([oracle.quantize_row_q8(w[r * cols:(r + 1) * cols])
                             for r in range(rows)])
        gq = np.zeros_like(wq)
        for r in range(rows):
            seg = np.zeros(cols // 32 * 36, np.uint8)
            L.mia_quantize_row_q8(w[r * cols:].ctypes.data, seg.ctypes.data, cols)
            gq[r * seg.size:(r + 1) * seg.size] = seg
        assert np.array_equal(gq, wq), "quantize %dx%d" % (rows, cols)
        out = np.zeros(rows, np.float32)
        xq = np.zeros(cols // 32 * 36, np.uint8)
        L.mia_matvec(out.ctypes.data, wq.ctypes.data, 1, x.ctypes.data, xq.ctypes.data, rows, cols)
        assert_bits(out, oracle.matvec(wq, 1, x, rows, cols), "q8 matvec %dx%d" % (rows, cols))
        assert np.array_equal(xq, oracle.quantize_row_q8(x))
        # F32 rows
        L.mia_matvec(out.ctypes.data, w.ctypes.data, 0, x.ctypes.data, None, rows, cols)
        assert_bits(out, oracle.matvec(w, 0, x, rows, cols), "f32 matvec %dx%d" % (rows, cols))
        # dequantize
        deq = np.zeros(cols, np.float32)
        L.mia_dequantize_row(1, wq.ctypes.data, deq.ctypes.data, cols)
        assert_bits(deq, oracle.dequantize_row_q8(wq[: cols // 32 * 36], cols), "dequantize")
    assert L.mia_tensor_error() is None  # no op of this test failed


def test_matvec_registered_weights(oracle):
    """A registered matrix is read from its HBM copy: bit-equal results;
    another shape at the same pointer is not served from the copy; after
    unregistering, the host bytes are read again."""
    say("test_matvec_registered_weights")
    L = M.lib()
    rows, cols = 1024, 512
    u = _xorshift_uniform(rows * cols + cols, state=0x2468ACE)
    w = (u[: rows * cols] * 2.0).astype(np.float32)
    x = u[rows * cols:].copy()
    wq = oracle.quantize_row_q8(w)
    out = np.zeros(rows, np.float32)
    assert L.mia_matvec_register(wq.ctypes.data, 1, rows, cols) == 0
    assert L.mia_matvec_register(w.ctypes.data, 0, rows, cols) == 0
    for _ in range(2):
        L.mia_matvec(out.ctypes.data, wq.ctypes.data, 1, x.ctypes.data, None, rows, cols)
        assert_bits(out, oracle.matvec(wq, 1, x, rows, cols), "registered q8")
        L.mia_matvec(out.ctypes.data, w.ctypes.data, 0, x.ctypes.data, None, rows, cols)
        assert_bits(out, oracle.matvec(w, 0, x, rows, cols), "registered f32")
    half = np.zeros(rows // 2, np.float32)
    L.mia_matvec(half.ctypes.data, wq.ctypes.data, 1, x.ctypes.data, None, rows // 2, cols)
    assert_bits(half, oracle.matvec(wq, 1, x, rows // 2, cols), "other shape, same pointer")
    assert L.mia_matvec_unregister(wq.ctypes.data) == 0
    assert L.mia_matvec_unregister(wq.ctypes.data) == -1
    assert L.mia_matvec_unregister(w.ctypes.data) == 0
    wq[4:36] = oracle.quantize_row_q8(np.ones(32, np.float32))[4:]  # new codes in row 0
    L.mia_matvec(out.ctypes.data, wq.ctypes.data, 1, x.ctypes.data, None, rows, cols)
    assert_bits(out, oracle.matvec(wq, 1, x, rows, cols), "after unregistering")
    assert L.mia_matvec_register(wq.ctypes.data, 1, rows, 33) == -1  # cols % 32


# ---- expert table ------------------------------------------------------------------

def test_table_synth_matches_host_generator(oracle, qwen_dims, qwen_moe):
    say("test_table_synth_matches_host_generator")
    for (l, e) in [(0, 0), (0, 77), (1, 127)]:
        got = qwen_moe.read_expert(l, e)
        want = oracle.synth_expert_blob(W.WEIGHT_SEED, l, e, qwen_dims)
        assert np.array_equal(got, want), "expert (%d,%d)" % (l, e)


def test_loader_port_roundtrip_and_failure(oracle, tiny_dims):
    say("test_loader_port_roundtrip_and_failure")
    shape = dict(oracle.TINY)
    moe = M.Moe(n_layers=2, max_tokens=8, device=0, **shape)
    try:
        blobs = {(l, e): oracle.synth_expert_blob(1000 + l, l, e, tiny_dims)
                 for l in range(2) for e in range(tiny_dims.n_experts)}
        calls = []

        def load(l, e, dst):
            calls.append((l, e))
            b = blobs[(l, e)]
            ctypes.memmove(dst, b.ctypes.data, b.size)
            return 0

        moe.load_experts(load)
        assert len(calls) == 2 * tiny_dims.n_experts
        for (l, e), b in blobs.items():
            assert np.array_equal(moe.read_expert(l, e), b)

        def failing(l, e, dst):
            return -1 if (l, e) == (1, 3) else load(l, e, dst)

        with pytest.raises(RuntimeError, match="layer 1 expert 3"):
            moe.load_experts(failing)
        # nothing loaded before the failure was poisoned
        assert np.array_equal(moe.read_expert(1, 2), blobs[(1, 2)])
    finally:
        moe.close()


# ---- single layer --------------------------------------------------------------------

def _gpu_layer(moe, layer, x, bias, flags):
    moe.set_flags(flags)
    try:
        return moe.layer(layer, x, bias=bias)
    finally:
        moe.set_flags(0)


def _compare_layer(O, moe, d, layer, x, router, bias=None, label="", matrix=False):
    """Vector path against the oracle; with matrix=True also the default
    (matrix-core) path of the same call (bit-equal) and the MHIP_FAST_DOWN
    option (routing bit-equal, output within TOL)."""
    xg, idx, w, logits = _gpu_layer(moe, layer, x, bias, M.MHIP_EXACT_EXPERTS)
    xo, io, wo, lo, _ = oracle_layer(O, moe, d, layer, x, router, bias=bias,
                                    need=idx.ravel().tolist())
    say("  %s exact path: rel err %.3e" % (label, rel_err(xg - x, xo - x)))
    assert np.array_equal(idx, io), "%s: expert indices differ" % label
    assert_bits(logits, lo, label + " logits")
    assert_bits(w, wo, label + " gate weights")
    assert_bits(xg, xo, label + " layer output")
    if matrix:
        n0 = M.lib().mhip_matrix_layers(moe.gpu)
        xm, im, wm, lm = _gpu_layer(moe, layer, x, bias, 0)
        assert M.lib().mhip_matrix_layers(moe.gpu) == n0 + 1, "%s: matrix path not taken" % label
        say("  %s matrix-core path: bit-equal" % label)
        assert np.array_equal(im, io), "%s: matrix path expert indices differ" % label
        assert_bits(lm, lo, label + " matrix path logits")
        assert_bits(wm, wo, label + " matrix path gate weights")
        assert_bits(xm, xo, label + " matrix path layer output")
        xf, i_f, wf, lf = _gpu_layer(moe, layer, x, bias, M.MHIP_FAST_DOWN)
        assert M.lib().mhip_matrix_layers(moe.gpu) == n0 + 2, "%s: matrix path not taken" % label
        e_delta, e_out = rel_err(xf - x, xo - x), rel_err(xf, xo)
        say("  %s fused-down option: rel err update %.3e, output %.3e" % (label, e_delta, e_out))
        assert np.array_equal(i_f, io), "%s: fused-down expert indices differ" % label
        assert_bits(wf, wo, label + " fused-down gate weights")
        assert e_delta <= TOL and e_out <= TOL, label
    return idx


@pytest.mark.parametrize("T", [1, 4, 64])
def test_layer_decode_shapes(oracle, qwen_dims, qwen_moe, T):
    say("test_layer_decode_shapes T=%d" % T)
    x = oracle.synth_x(W.X_SEED, T, qwen_dims.dim)
    router = oracle.synth_router(W.WEIGHT_SEED, 0, qwen_dims)
    _compare_layer(oracle, qwen_moe, qwen_dims, 0, x, router, label="T=%d" % T)


def test_layer_vector_path_255_with_bias(oracle, qwen_dims, qwen_moe):
    """The most tokens the one-launch rmsnorm + router + selection front takes
    (255 x 8 assignments stay below the matrix-core threshold), with the
    skewed logit bias: bit-exact with and without MHIP_EXACT_EXPERTS."""
    say("test_layer_vector_path_255_with_bias")
    x = oracle.synth_x(W.X_SEED + 21, 255, qwen_dims.dim)
    router = oracle.synth_router(W.WEIGHT_SEED, 0, qwen_dims)
    bias = W.zipf_bias(qwen_dims.n_experts)
    _compare_layer(oracle, qwen_moe, qwen_dims, 0, x, router, bias=bias, label="T=255 bias")
    n0 = M.lib().mhip_matrix_layers(qwen_moe.gpu)
    xg, idx, w, logits = _gpu_layer(qwen_moe, 0, x, bias, 0)
    assert M.lib().mhip_matrix_layers(qwen_moe.gpu) == n0, "T=255 took the matrix path"
    xo, io, wo, lo, _ = oracle_layer(oracle, qwen_moe, qwen_dims, 0, x, router, bias=bias,
                                    need=idx.ravel().tolist())
    assert np.array_equal(idx, io)
    assert_bits(logits, lo, "T=255 default path logits")
    assert_bits(w, wo, "T=255 default path gate weights")
    assert_bits(xg, xo, "T=255 default path layer output")


def test_layer_prefill_512(oracle, qwen_dims, qwen_moe):
    say("test_layer_prefill_512")
    x = oracle.synth_x(W.X_SEED, 512, qwen_dims.dim)
    router = oracle.synth_router(W.WEIGHT_SEED, 1, qwen_dims)
    idx = _compare_layer(oracle, qwen_moe, qwen_dims, 1, x, router, label="T=512", matrix=True)
    cnt = np.bincount(idx.ravel(), minlength=128)
    assert cnt.min() > 0  # near-uniform load touches every expert


def test_layer_skewed_2048(oracle, qwen_dims, qwen_moe):
    say("test_layer_skewed_2048")
    x = oracle.synth_x(W.X_SEED, 2048, qwen_dims.dim)
    router = oracle.synth_router(W.WEIGHT_SEED, 0, qwen_dims)
    bias = W.zipf_bias(qwen_dims.n_experts)
    idx = _compare_layer(oracle, qwen_moe, qwen_dims, 0, x, router, bias=bias, label="skew",
                         matrix=True)
    cnt = np.sort(np.bincount(idx.ravel(), minlength=128))[::-1]
    share4 = cnt[:4].sum() / cnt.sum()
    zero = int((cnt == 0).sum())
    say("  top-4 share %.3f, %d experts idle" % (share4, zero))
    assert 0.35 < share4 < 0.5 and 20 <= zero <= 40


def _every_token(oracle, d, T, seed, bias=None):
    """One matrix-core layer at T tokens on a fresh one-layer handle with a
    non-unit ffn_norm: every token's logits, expert indices, gate weights and
    layer output bit-equal to the oracle's (its expert-bucketed layer, same
    bits as its per-token one)."""
    moe = M.Moe(n_layers=1, max_tokens=T, device=0, **W.SHAPE)
    try:
        moe.synth(W.WEIGHT_SEED)
        router = oracle.synth_router(W.WEIGHT_SEED, 0, d)
        norm = (1.0 + 0.1 * np.random.default_rng(77).standard_normal(d.dim)).astype(np.float32)
        moe.set_layer(0, norm, router)
        moe.sync()
        x = oracle.synth_x(seed, T, d.dim)
        xm, im, wm, lm = _gpu_layer(moe, 0, x, bias, 0)
        blobs = [None] * d.n_experts
        for e in sorted(set(im.ravel().tolist())):
            blobs[e] = moe.read_expert(0, e)
        xo, io, wo, lo = oracle.moe_layer_bucketed(d, x, norm, router, blobs, bias=bias,
                                                   nthreads=NTHREADS)
        assert_bits(lm, lo, "logits")
        assert np.array_equal(im, io), "expert indices"
        assert_bits(wm, wo, "gate weights")
        assert_bits(xm, xo, "layer output")
        say("  all %d tokens bit-equal" % T)
    finally:
        moe.close()


def test_layer_prefill_4096_every_token(oracle, qwen_dims):
    """T=4096, the prefill benchmark shape (matrix-core experts, four router
    chains per lane)."""
    say("test_layer_prefill_4096_every_token")
    _every_token(oracle, qwen_dims, 4096, W.X_SEED + 11)


def test_layer_ragged_2111_with_bias(oracle, qwen_dims):
    """T=2111: the last 64-token router group and the last bucket tiles are
    partial, four router chains per lane, with the skewed logit bias."""
    say("test_layer_ragged_2111_with_bias")
    _every_token(oracle, qwen_dims, 2111, W.X_SEED + 13, bias=W.zipf_bias(qwen_dims.n_experts))


def test_matrix_path_ragged_buckets(oracle, qwen_dims, qwen_moe):
    """T=300: 2400 assignments (above the matrix-core threshold), every
    expert bucket smaller than one 128-row tile; the tile table must count
    ceil(bucket / 128) tiles per non-empty expert."""
    say("test_matrix_path_ragged_buckets")
    T = 300
    assert T * qwen_dims.n_active >= M.GEMM_MIN_A
    x = oracle.synth_x(W.X_SEED + 3, T, qwen_dims.dim)
    router = oracle.synth_router(W.WEIGHT_SEED, 0, qwen_dims)
    xm, im, wm, lm = _gpu_layer(qwen_moe, 0, x, None, 0)
    sc = qwen_moe.scratch()
    E = qwen_dims.n_experts
    groups = qwen_moe.d2h(sc.groups, 1 + 3 * E, np.int32)
    gtile = qwen_moe.d2h(sc.gtile, E + 1, np.int32)
    G = int(groups[0])
    sizes = groups[3:3 + 3 * G:3] - groups[2:2 + 3 * G:3]
    assert sizes.sum() == T * qwen_dims.n_active and sizes.max() < 128
    assert np.array_equal(gtile[:G + 1], np.concatenate([[0], np.cumsum((sizes + 127) // 128)]))
    # light tiles: a bucket's last tile when it holds at most 64 rows
    glight = qwen_moe.d2h(sc.glight, E + 1, np.int32)
    rem = sizes % 128
    assert np.array_equal(glight[:G + 1],
                          np.concatenate([[0], np.cumsum((rem != 0) & (rem <= 64))]))
    xo, io, wo, lo, _ = oracle_layer(oracle, qwen_moe, qwen_dims, 0, x, router,
                                    need=im.ravel().tolist())
    assert np.array_equal(im, io)
    assert_bits(wm, wo, "gate weights")
    assert_bits(xm, xo, "layer output")


def test_dispatch_matches_oracle(oracle, qwen_dims, qwen_moe):
    say("test_dispatch_matches_oracle")
    x = oracle.synth_x(W.X_SEED + 1, 300, qwen_dims.dim)
    _, idx, _, _ = qwen_moe.layer(0, x)
    sc = qwen_moe.scratch()
    E, A = qwen_dims.n_experts, idx.size
    counts = qwen_moe.d2h(sc.counts, E, np.int32)
    offsets = qwen_moe.d2h(sc.offsets, E + 1, np.int32)
    perm = qwen_moe.d2h(sc.perm, A, np.int32)
    pos = qwen_moe.d2h(sc.pos, A, np.int32)
    c, o, p, q = oracle.dispatch(idx, E)
    assert np.array_equal(counts, c) and np.array_equal(offsets, o)
    assert np.array_equal(perm, p) and np.array_equal(pos, q)


def test_forced_sequential_rmsnorm_same_bits(oracle, qwen_dims, qwen_moe):
    say("test_forced_sequential_rmsnorm_same_bits")
    x = oracle.synth_x(W.X_SEED + 2, 16, qwen_dims.dim)
    a = qwen_moe.layer(0, x)
    qwen_moe.set_flags(M.MHIP_FORCE_SEQ_RMS)
    try:
        b = qwen_moe.layer(0, x)
    finally:
        qwen_moe.set_flags(0)
    st = qwen_moe.status()  # the status words describe the last call
    assert st[1] == 16 and st[3] == 1, st
    for u, v in zip(a, b):
        assert np.array_equal(np.asarray(u).view(np.uint32), np.asarray(v).view(np.uint32))


def test_zero_tokens_and_limits(qwen_moe):
    say("test_zero_tokens_and_limits")
    x = np.zeros((0, 2048), np.float32)
    assert M.lib().mia_moe_layer(qwen_moe.h, 0, x.ctypes.data, 0) == 0
    big = np.zeros((2049, 2048), np.float32)
    with pytest.raises(RuntimeError, match="max_tokens"):
        qwen_moe.layer(0, big)
    with pytest.raises(RuntimeError, match="layer 5"):
        qwen_moe.layer(5, np.zeros((1, 2048), np.float32))


# ---- tiny model (the reference's e2e shape) and edge cases ----------------------------

def _tiny_handle(oracle, d, layers=1, max_tokens=64, seed=5):
    moe = M.Moe(n_layers=layers, max_tokens=max_tokens, device=0,
                **dict(oracle.TINY, n_experts=d.n_experts, n_active=d.n_active))
    routers = []
    for l in range(layers):
        for e in range(d.n_experts):
            moe.load_expert(l, e, oracle.synth_expert_blob(seed, l, e, d))
        r = oracle.synth_router(seed, l, d) * np.float32(20.0)
        moe.set_layer(l, np.ones(d.dim, np.float32), r)
        routers.append(r)
    return moe, routers


@pytest.mark.parametrize("E,K", [(8, 2), (8, 1), (8, 8), (64, 6)])
def test_layer_tiny_shapes(oracle, E, K):
    say("test_layer_tiny_shapes E=%d K=%d" % (E, K))
    d = oracle.dims(**dict(oracle.TINY, n_experts=E, n_active=K))
    moe, routers = _tiny_handle(oracle, d)
    try:
        x = oracle.synth_x(11, 64, d.dim)
        _compare_layer(oracle, moe, d, 0, x, routers[0], label="tiny E=%d K=%d" % (E, K))
    finally:
        moe.close()


def test_router_ties_lowest_index_first(oracle):
    say("test_router_ties_lowest_index_first")
    d = oracle.dims(**oracle.TINY)
    moe, routers = _tiny_handle(oracle, d)
    try:
        r = routers[0].copy()
        r[5] = r[1]
        r[6] = r[1]  # three experts with identical logits
        moe.set_layer(0, np.ones(d.dim, np.float32), r)
        x = oracle.synth_x(12, 32, d.dim)
        idx = _compare_layer(oracle, moe, d, 0, x, r, label="ties")
        for t in range(idx.shape[0]):
            row = idx[t].tolist()
            tied = [e for e in row if e in (1, 5, 6)]
            assert tied == sorted(tied)
    finally:
        moe.close()


# ---- stacks ------------------------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 64])
def test_stack_matches_oracle_layer_by_layer(oracle, qwen_dims, qwen_moe, T):
    say("test_stack_matches_oracle_layer_by_layer T=%d" % T)
    x0 = oracle.synth_x(W.X_SEED + 3, T, qwen_dims.dim)
    xg = qwen_moe.stack(0, 2, x0)
    x = x0
    for l in range(2):
        router = oracle.synth_router(W.WEIGHT_SEED, l, qwen_dims)
        x, _, _, _, _ = oracle_layer(oracle, qwen_moe, qwen_dims, l, x, router)
    assert_bits(xg, x, "2-layer stack T=%d" % T)
