"""The CPU oracle against the reference's own known answers, invariants and
tolerances (tests/*.c and tools/internal/**/_test.go of the reference), plus
brute force where the mathematics fixes the answer."""
import numpy as np
import pytest

from helpers import xorshift_uniform


# ---- Q8_0 (tests/test_quant.c, tools/internal/mia/format_test.go) -------------

def test_row_bytes_by_type(oracle):
    L = oracle.lib()
    assert L.orc_row_bytes(0, 64) == 256
    assert L.orc_row_bytes(1, 64) == 2 * 36


def test_q8_roundtrip_error_is_bounded(oracle):
    x = (xorshift_uniform(256) * np.float32(3.0)).astype(np.float32)
    q = oracle.quantize_row_q8(x)
    y = oracle.dequantize_row_q8(q, 256)
    for b in range(8):
        d = q[b * 36: b * 36 + 4].view(np.float32)[0]
        assert np.all(np.abs(x[b * 32:(b + 1) * 32] - y[b * 32:(b + 1) * 32]) <= d * 0.5 + 1e-7)


def test_q8_zero_block_is_exact(oracle):
    q = oracle.quantize_row_q8(np.zeros(32, np.float32))
    assert q[:4].view(np.float32)[0] == 0.0
    assert not oracle.dequantize_row_q8(q, 32).any()


def test_q8_max_maps_to_127_and_halves_round_away(oracle):
    x = np.zeros(32, np.float32)
    x[3], x[7] = -2.0, 1.0
    q = oracle.quantize_row_q8(x)[4:].view(np.int8)
    assert q[3] == -127 and q[7] == 64  # round(63.5) = 64


def test_q8_matches_closed_form_on_exact_grid(oracle):
    # Values k*d with |k| <= 127 and amax = 127*d quantize to exactly k.
    rng = np.random.default_rng(0)
    k = rng.integers(-127, 128, size=32)
    k[0] = 127
    d = np.float32(0.25)
    q = oracle.quantize_row_q8((k * d).astype(np.float32))
    assert q[:4].view(np.float32)[0] == d
    assert np.array_equal(q[4:].view(np.int8), k.astype(np.int8))


# ---- mat-vec (tests/test_matmul.c) ----------------------------------------------

def _naive(w, x, rows, cols):
    return w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)


@pytest.mark.parametrize("rows,cols", [(7, 32), (1024, 512)])
def test_f32_matvec_close_to_double(oracle, rows, cols):
    u = xorshift_uniform(rows * cols + cols, state=0x1234567)
    w, x = u[: rows * cols], u[rows * cols:]
    out = oracle.matvec(w, 0, x, rows, cols)
    assert np.max(np.abs(out - _naive(w, x, rows, cols))) <= 1e-3


@pytest.mark.parametrize("rows,cols", [(5, 64), (2048, 768)])
def test_q8_matvec_close_to_double(oracle, rows, cols):
    u = xorshift_uniform(rows * cols + cols, state=0x7654321)
    w, x = u[: rows * cols], u[rows * cols:]
    wq = np.concatenate([oracle.quantize_row_q8(w[r * cols:(r + 1) * cols]) for r in range(rows)])
    out = oracle.matvec(wq, 1, x, rows, cols)
    assert np.max(np.abs(out - _naive(w, x, rows, cols))) <= 0.02 * np.sqrt(cols)


def test_q8_matvec_integer_closed_form(oracle):
    # With scales that are powers of two every term is exact, so the result
    # is sum_b d_w d_x sum_i q_w q_x computed in exact arithmetic.
    rng = np.random.default_rng(1)
    rows, cols = 9, 128
    qw = rng.integers(-127, 128, size=(rows, cols))
    qw[:, ::32] = 127
    dw = np.float32(2.0 ** -7)
    x = (rng.integers(-127, 128, size=cols) * np.float32(2.0 ** -5)).astype(np.float32)
    x[::32] = np.float32(127 * 2.0 ** -5)
    wq = np.concatenate([oracle.quantize_row_q8((qw[r] * dw).astype(np.float32))
                         for r in range(rows)])
    out = oracle.matvec(wq, 1, x, rows, cols)
    exact = (qw.astype(np.float64) * float(dw)) @ (x.astype(np.float64))
    assert np.array_equal(out.astype(np.float64), exact)


# ---- routing (tools/internal/ref/ref_test.go, src/model/forward.c:95-114) ---------

def test_topk_routing_known_answer(oracle):
    idx, w, _ = oracle.route([0, 3, 1, 2], 2, norm_topk=1)
    assert idx.tolist() == [1, 3]
    assert abs(float(w.sum()) - 1.0) < 1e-6
    idx, w, _ = oracle.route([0, 3, 1, 2], 2, norm_topk=0)
    assert idx.tolist() == [1, 3]
    assert abs(float(w.sum()) - 1.0) > 1e-3


def test_topk_ties_pick_lowest_index_brute_force(oracle):
    rng = np.random.default_rng(2)
    for trial in range(200):
        E = int(rng.integers(2, 40))
        K = int(rng.integers(1, E + 1))
        p = rng.integers(0, 5, size=E).astype(np.float32) / np.float32(7.0)
        got = oracle.top_k(p, K).tolist()
        want = sorted(range(E), key=lambda i: (-float(p[i]), i))[:K]
        assert got == want, (p, K)


def test_softmax_is_a_distribution(oracle):
    rng = np.random.default_rng(3)
    l = rng.normal(size=128).astype(np.float32)
    p = oracle.softmax(l)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
    assert np.array_equal(np.argsort(-p, kind="stable"), np.argsort(-l, kind="stable"))


def test_rmsnorm_unit_weight_gives_unit_rms(oracle):
    out = oracle.rmsnorm(np.array([1, -2, 3, 4], np.float32), np.ones(4, np.float32), 0.0)
    assert abs(float(np.sqrt(np.mean(out.astype(np.float64) ** 2))) - 1.0) < 1e-5


def test_identical_experts_make_output_router_independent(oracle, tiny_dims):
    d = tiny_dims
    blob = oracle.synth_expert_blob(9, 0, 0, d)
    blobs = [blob] * d.n_experts
    x = oracle.synth_x(4, 16, d.dim)
    router = oracle.synth_router(9, 0, d)
    norm = np.ones(d.dim, np.float32)
    a = oracle.moe_layer(d, x, norm, router, blobs)[0]
    b = oracle.moe_layer(d, x, norm, (router * np.float32(-3.0)).astype(np.float32), blobs)[0]
    assert np.max(np.abs(a - b)) <= 1e-4


def test_threads_do_not_change_bits(oracle, tiny_dims):
    d = tiny_dims
    blobs = [oracle.synth_expert_blob(3, 0, e, d) for e in range(d.n_experts)]
    x = oracle.synth_x(6, 64, d.dim)
    router = oracle.synth_router(3, 0, d)
    norm = np.ones(d.dim, np.float32)
    a = oracle.moe_layer(d, x, norm, router, blobs, nthreads=1)
    b = oracle.moe_layer(d, x, norm, router, blobs, nthreads=4)
    for u, v in zip(a, b):
        assert np.array_equal(np.asarray(u).view(np.uint32), np.asarray(v).view(np.uint32))


def test_missing_expert_fails_like_a_failed_load(oracle, tiny_dims):
    d = tiny_dims
    x = oracle.synth_x(4, 1, d.dim)
    with pytest.raises(RuntimeError):
        oracle.moe_layer(d, x, np.ones(d.dim, np.float32), oracle.synth_router(9, 0, d),
                         [None] * d.n_experts)


# ---- dispatch ---------------------------------------------------------------------

def test_dispatch_is_the_stable_bucketing(oracle):
    rng = np.random.default_rng(4)
    for T, K, E in [(1, 8, 128), (37, 2, 8), (300, 8, 128), (64, 6, 64)]:
        idx = np.stack([rng.choice(E, size=K, replace=False) for _ in range(T)]).astype(np.int32)
        counts, offsets, perm, pos = oracle.dispatch(idx, E)
        want = sorted(range(T * K), key=lambda a: (int(idx.ravel()[a]), a))
        assert perm.tolist() == want
        assert np.array_equal(counts, np.bincount(idx.ravel(), minlength=E))
        assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
        assert np.array_equal(pos[perm], np.arange(T * K))


# ---- synthetic generator ------------------------------------------------------------

def test_synthetic_normals_have_unit_moments(oracle):
    x = oracle.synth_x(123, 64, 2048).astype(np.float64).ravel()
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert abs(np.mean(x ** 4) / np.mean(x ** 2) ** 2 - 3.0) < 0.1  # normal kurtosis
    assert np.array_equal(x, oracle.synth_x(123, 64, 2048).astype(np.float64).ravel())


def test_synthetic_blob_layout(oracle, tiny_dims):
    d = tiny_dims
    b = oracle.synth_expert_blob(1, 0, 2, d)
    assert b.size == oracle.blob_bytes(d) and b.size % 16384 == 0
    rb = d.dim // 32 * 36
    assert oracle.off_up(d) == d.expert_hidden * rb
    # padding past the down matrix stays zero
    end = oracle.off_down(d) + d.dim * (d.expert_hidden // 32 * 36)
    assert not b[end:].any()


# ---- the bucketed layer, routing only, and the 64-row-chunk split ---------------

MID = dict(dim=512, n_experts=16, n_active=4, expert_hidden=256, norm_topk=1, norm_eps=1e-6)


def _weights(oracle, d, seed, sigma_norm=0.1):
    blobs = [oracle.synth_expert_blob(seed, 0, e, d) for e in range(d.n_experts)]
    router = (oracle.synth_router(seed, 0, d) * np.float32(10.0)).astype(np.float32)
    rng = np.random.default_rng(seed)
    norm = (1.0 + sigma_norm * rng.standard_normal(d.dim)).astype(np.float32)
    return blobs, router, norm


def _same_bits(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.mark.parametrize("shape,T,with_bias", [("tiny", 64, False), ("tiny", 1, True),
                                               ("mid", 97, True), ("mid8", 40, False)])
def test_bucketed_layer_is_bit_equal(oracle, shape, T, with_bias):
    kw = {"tiny": oracle.TINY, "mid": MID, "mid8": dict(MID, n_experts=64, n_active=8)}[shape]
    d = oracle.dims(**kw)
    blobs, router, norm = _weights(oracle, d, 21)
    x = oracle.synth_x(22, T, d.dim)
    bias = (np.random.default_rng(2).standard_normal(d.n_experts)).astype(np.float32) \
        if with_bias else None
    xa, ia, wa, la, _ = oracle.moe_layer(d, x, norm, router, blobs, bias=bias)
    xb, ib, wb, lb = oracle.moe_layer_bucketed(d, x, norm, router, blobs, bias=bias, nthreads=4)
    assert np.array_equal(ia, ib)
    assert _same_bits(wa, wb) and _same_bits(la, lb)
    assert _same_bits(xa, xb)
    ir, wr, lr = oracle.route_tokens(d, x, norm, router, bias=bias, nthreads=3)
    assert np.array_equal(ia, ir) and _same_bits(wa, wr) and _same_bits(la, lr)


def test_bucketed_layer_missing_expert_fails(oracle):
    d = oracle.dims(**oracle.TINY)
    blobs, router, norm = _weights(oracle, d, 5)
    x = oracle.synth_x(4, 8, d.dim)
    _, idx, _, _, _ = oracle.moe_layer(d, x, norm, router, blobs)
    blobs[int(idx[0, 0])] = None
    with pytest.raises(RuntimeError):
        oracle.moe_layer_bucketed(d, x, norm, router, blobs)


def test_row_chunk_threads_do_not_change_bits(oracle):
    """One token with nthreads > 1 splits every large matrix into 64-row
    chunks over threads (the reference's CHUNK_ROWS split): same bits."""
    d = oracle.dims(**MID)
    blobs, router, norm = _weights(oracle, d, 31)
    x = oracle.synth_x(32, 1, d.dim)
    a = oracle.moe_layer(d, x, norm, router, blobs, nthreads=1)
    b = oracle.moe_layer(d, x, norm, router, blobs, nthreads=4)
    for u, v in zip(a, b):
        assert _same_bits(u, v)


# ---- where the logit bias enters (added after the router product, before the
# softmax; the hook the skewed workload adds to forward.c:175-176) --------------

def test_bias_is_added_to_the_router_logits(oracle):
    d = oracle.dims(**MID)
    blobs, router, norm = _weights(oracle, d, 41)
    x = oracle.synth_x(42, 8, d.dim)
    bias = np.random.default_rng(3).standard_normal(d.n_experts).astype(np.float32)
    _, _, _, l0, _ = oracle.moe_layer(d, x, norm, router, blobs)
    _, _, _, l1, _ = oracle.moe_layer(d, x, norm, router, blobs, bias=bias)
    assert _same_bits(l1, (l0 + bias).astype(np.float32))  # one fp32 add per logit


def test_dominant_bias_forces_rank_zero(oracle):
    d = oracle.dims(**MID)
    blobs, router, norm = _weights(oracle, d, 43)
    x = oracle.synth_x(44, 16, d.dim)
    for e in (0, 7, d.n_experts - 1):
        bias = np.zeros(d.n_experts, np.float32)
        bias[e] = 100.0
        _, idx, w, _, _ = oracle.moe_layer(d, x, norm, router, blobs, bias=bias)
        assert np.all(idx[:, 0] == e)
        # the other experts' softmax mass underflows next to e^100: w_0 = 1
        assert np.all(w[:, 0] == np.float32(1.0))


def test_constant_bias_keeps_the_ranking(oracle):
    d = oracle.dims(**MID)
    blobs, router, norm = _weights(oracle, d, 45)
    x = oracle.synth_x(46, 32, d.dim)
    _, i0, w0, l0, _ = oracle.moe_layer(d, x, norm, router, blobs)
    for c in (-3.0, 0.5, 7.0):
        _, i1, w1, _, _ = oracle.moe_layer(d, x, norm, router, blobs,
                                           bias=np.full(d.n_experts, c, np.float32))
        # a constant shift moves every logit by one rounding at most: the
        # ranking is unchanged wherever its gaps exceed that rounding
        srt = np.sort(l0, axis=1)[:, ::-1]
        gap = np.min(np.abs(np.diff(srt[:, :d.n_active + 1], axis=1)), axis=1)
        clear = gap > 4 * np.spacing(np.float32(abs(c) + np.max(np.abs(l0))))
        assert clear.sum() >= 28
        assert np.array_equal(i0[clear], i1[clear])
        assert np.max(np.abs(w0 - w1)) < 1e-5


def test_native_build_gives_the_same_bits(oracle):
    """The -march=native build of the oracle (the best-case CPU baseline) is
    the same arithmetic: -ffp-contract=off keeps every product rounded."""
    import subprocess
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run(["make", "-s", "-C", os.path.join(root, "oracle"), "native"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("native oracle build failed: %s" % r.stderr[-200:])
    d = oracle.dims(**MID)
    blobs, router, norm = _weights(oracle, d, 51)
    x = oracle.synth_x(52, 24, d.dim)
    a = oracle.moe_layer(d, x, norm, router, blobs)
    b1 = oracle.moe_layer(d, x[:1], norm, router, blobs, nthreads=4)
    try:
        oracle.select("native")
        b = oracle.moe_layer(d, x, norm, router, blobs)
        c1 = oracle.moe_layer(d, x[:1], norm, router, blobs, nthreads=4)
    finally:
        oracle.select("default")
    for u, v in zip(a, b):
        assert _same_bits(u, v)
    for u, v in zip(b1, c1):
        assert _same_bits(u, v)
