"""GPU parity of the persistent decode-stack kernel (one token, many layers).

By default the kernel's router is exact (the certified ranking, the
reference's sequential logit chains for the gate weights): every layer's
indices, gate weights and output are bit-equal to the oracle's. With
MHIP_DECODE_CERTIFIED the gate weights come from the parallel logits:
indices bit-equal, outputs within the north-star tolerance
(max|diff| / max|ref| <= 1e-3; ~1e-6 is expected).
"""
import ctypes
import sys

import numpy as np
import pytest

import motoria_amd as M
from motoria_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-3
LAYERS = 6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.fixture(scope="module")
def moe():
    say("open decode handle: %d layers" % LAYERS)
    m = M.Moe(n_layers=LAYERS, max_tokens=4, device=0, **W.SHAPE)
    m.synth(W.WEIGHT_SEED)
    m.sync()
    yield m
    m.close()


def run_oracle_layer(O, moe, d, layer, x, bias=None):
    router = O.synth_router(W.WEIGHT_SEED, layer, d)
    norm = np.ones(d.dim, np.float32)
    x1 = np.array(x, np.float32).reshape(1, -1)
    # the oracle's own routing prologue tells which experts to fetch
    xn = O.rmsnorm(x1[0], norm, d.norm_eps)
    lg = O.matvec(router, 0, xn, d.n_experts, d.dim)
    if bias is not None:
        lg = (lg + bias).astype(np.float32)
    idx, _, _ = O.route(lg, d.n_active)
    blobs = [None] * d.n_experts
    for e in idx.tolist():
        blobs[e] = moe.read_expert(layer, e)
    return O.moe_layer(d, x1, norm, router, blobs, bias=bias)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("certified", [False, True])
def test_decode_layer_by_layer_matches_oracle(oracle, qwen_dims, moe, certified):
    say("test_decode_layer_by_layer_matches_oracle certified=%d" % certified)
    d = qwen_dims
    x = oracle.synth_x(W.X_SEED, 1, d.dim)[0]
    worst = 0.0
    moe.set_flags(M.MHIP_DECODE_CERTIFIED if certified else 0)
    try:
        for l in range(LAYERS):
            xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, l, x)
            xg, ig, wg = moe.decode(l, l + 1, x)
            st = moe.decode_status()
            assert st[0] == 0, "decode aborted: %s" % st
            assert np.array_equal(ig[0], io[0]), "layer %d: expert indices %s vs %s" % (
                l, ig[0], io[0])
            e_out = rel(xg - x, xo[0] - x)
            e_w = rel(wg[0], wo[0])
            worst = max(worst, e_out)
            say("  layer %d: idx %s  rel err delta %.2e  w %.2e  status %s"
                % (l, ig[0].tolist(), e_out, e_w, st))
            if certified:
                assert e_out <= TOL and e_w <= TOL
            else:
                assert np.array_equal(bits(wg[0]), bits(wo[0])), "layer %d gate weights" % l
                assert np.array_equal(bits(xg), bits(xo[0])), "layer %d output" % l
            x = xo[0]
    finally:
        moe.set_flags(0)
    say("  worst rel err %.2e" % worst)


def test_decode_full_stack_matches_oracle(oracle, qwen_dims, moe):
    """One launch over LAYERS layers from x0 (default flags): the oracle's
    free-running chain from the same x0, bit for bit (routing, gate weights
    and output of every layer)."""
    say("test_decode_full_stack_matches_oracle")
    d = qwen_dims
    x0 = oracle.synth_x(W.X_SEED + 7, 1, d.dim)[0]
    xg, ig, wg = moe.decode(0, LAYERS, x0)
    assert moe.decode_status()[0] == 0
    x = x0
    for l in range(LAYERS):
        xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, l, x)
        assert np.array_equal(ig[l], io[0]), "layer %d routing differs" % l
        assert np.array_equal(bits(wg[l]), bits(wo[0])), "layer %d gate weights" % l
        x = xo[0]
    assert np.array_equal(bits(xg), bits(x)), "%d-layer output: rel err %.2e" % (
        LAYERS, rel(xg - x0, x - x0))


@pytest.mark.parametrize("chains_first", [False, True])
def test_decode_exact_router_is_bit_equal(oracle, qwen_dims, moe, chains_first):
    """The exact chains beside the expert stream (a certified ranking) and
    before it (the path of a ranking that is not certified)."""
    say("test_decode_exact_router_is_bit_equal chains_first=%d" % chains_first)
    d = qwen_dims
    x = oracle.synth_x(W.X_SEED + 11, 1, d.dim)[0]
    moe.set_flags(M.MHIP_FORCE_EXACT_ROUTER | (M.MHIP_DECODE_CHAINS_FIRST if chains_first else 0))
    try:
        for l in range(2):
            xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, l, x)
            xg, ig, wg = moe.decode(l, l + 1, x)
            st = moe.decode_status()
            assert st[0] == 0 and st[2] >= 1, st
            assert np.array_equal(ig[0], io[0])
            assert np.array_equal(wg[0].view(np.uint32), wo[0].view(np.uint32))
            assert np.array_equal(xg.view(np.uint32), xo[0].view(np.uint32)), \
                "layer %d rel err %.2e" % (l, rel(xg - x, xo[0] - x))
            x = xo[0]
    finally:
        moe.set_flags(0)


@pytest.mark.parametrize("chains_first", [False, True])
def test_decode_exact_router_stack_is_bit_equal(oracle, qwen_dims, moe, chains_first):
    """One launch over LAYERS layers under the exact router: the exact
    logits, weights and outputs of every layer carried to the next."""
    say("test_decode_exact_router_stack_is_bit_equal chains_first=%d" % chains_first)
    d = qwen_dims
    x0 = oracle.synth_x(W.X_SEED + 17, 1, d.dim)[0]
    moe.set_flags(M.MHIP_FORCE_EXACT_ROUTER | (M.MHIP_DECODE_CHAINS_FIRST if chains_first else 0))
    try:
        xg, ig, wg = moe.decode(0, LAYERS, x0)
        st = moe.decode_status()
    finally:
        moe.set_flags(0)
    assert st[0] == 0 and st[2] == LAYERS, st
    x = x0
    for l in range(LAYERS):
        xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, l, x)
        assert np.array_equal(ig[l], io[0]), "layer %d routing differs" % l
        assert np.array_equal(wg[l].view(np.uint32), wo[0].view(np.uint32)), "layer %d weights" % l
        x = xo[0]
    assert np.array_equal(xg.view(np.uint32), x.view(np.uint32))


def test_decode_forced_sequential_rmsnorm(oracle, qwen_dims, moe):
    say("test_decode_forced_sequential_rmsnorm")
    x = oracle.synth_x(W.X_SEED + 13, 1, qwen_dims.dim)[0]
    a = moe.decode(0, 3, x)
    moe.set_flags(M.MHIP_FORCE_SEQ_RMS)
    try:
        b = moe.decode(0, 3, x)
        assert moe.decode_status()[1] >= 3
    finally:
        moe.set_flags(0)
    for u, v in zip(a, b):
        assert np.array_equal(np.asarray(u).view(np.uint32), np.asarray(v).view(np.uint32))


def test_decode_with_bias_and_repeats(oracle, qwen_dims, moe):
    say("test_decode_with_bias_and_repeats")
    d = qwen_dims
    bias = W.zipf_bias(d.n_experts)
    x = oracle.synth_x(W.X_SEED + 17, 1, d.dim)[0]
    xo, io, _, _, _ = run_oracle_layer(oracle, moe, d, 0, x, bias=bias)
    for rep in range(3):  # repeated launches reuse the workspace
        xg, ig, _ = moe.decode(0, 1, x, bias=bias)
        assert np.array_equal(ig[0], io[0])
        assert np.array_equal(bits(xg), bits(xo[0])), "rel err %.2e" % rel(xg - x, xo[0] - x)


def test_host_layer_one_token_uses_decode_launch(oracle, qwen_dims, moe):
    """mia_moe_layer at T = 1 (no logits asked): one launch of the persistent
    kernel with the exact router, bit-equal to the oracle's layer."""
    say("test_host_layer_one_token_uses_decode_launch")
    d = qwen_dims
    K = d.n_active
    for l in (0, LAYERS - 1):
        x0 = oracle.synth_x(W.X_SEED + 21 + l, 1, d.dim)
        x = x0.copy()
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        rc = M.lib().mia_moe_layer_ex(moe.h, l, x.ctypes.data, 1, None, idx.ctypes.data,
                                      w.ctypes.data, None)
        assert rc == 0, M.lib().mia_moe_error(moe.h).decode()
        st = moe.decode_status()
        assert st[0] == 0 and st[2] == 1, "the layer did not run as an exact-router decode launch"
        xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, l, x0[0])
        assert np.array_equal(idx, io[0]), "layer %d indices" % l
        assert np.array_equal(w.view(np.uint32), wo[0].view(np.uint32)), "layer %d gate weights" % l
        assert np.array_equal(x[0].view(np.uint32), xo[0].view(np.uint32)), "layer %d output" % l



def test_decode_routing_many_tokens(oracle, qwen_dims, moe):
    """Certified routing over many inputs: 24 tokens through every layer of
    the handle, one launch per layer, each layer's expert indices bit-equal
    to the oracle's routing of the same input (rmsnorm, router product,
    softmax, top-8), with the layer's output as the next layer's input."""
    say("test_decode_routing_many_tokens")
    d = qwen_dims
    norm = np.ones(d.dim, np.float32)
    routers = [oracle.synth_router(W.WEIGHT_SEED, l, d) for l in range(LAYERS)]
    xs = oracle.synth_x(W.X_SEED + 101, 24, d.dim)
    checked = 0
    for t in range(xs.shape[0]):
        x = xs[t]
        for l in range(LAYERS):
            xn = oracle.rmsnorm(x, norm, d.norm_eps)
            lg = oracle.matvec(routers[l], 0, xn, d.n_experts, d.dim)
            io, _, _ = oracle.route(lg, d.n_active)
            xg, ig, _ = moe.decode(l, l + 1, x)
            assert moe.decode_status()[0] == 0
            assert np.array_equal(ig[0], io), "token %d layer %d: %s vs %s" % (t, l, ig[0], io)
            checked += 1
            x = np.asarray(xg, np.float32)
    say("  %d layer routings bit-equal, status %s" % (checked, moe.decode_status()))


def test_aborted_launch_falls_back_per_stage(oracle, qwen_dims, moe):
    """A decode launch that aborts (here forced from the host: every
    workgroup leaves after the start barrier, MHIP_DECODE_FORCE_ABORT) leaves
    the host x untouched, and both host entry points rerun the layers per
    stage: the one-token layer call and the multi-layer decode return the
    oracle's bits, while the decode status still shows the aborted launch."""
    say("test_aborted_launch_falls_back_per_stage")
    d = qwen_dims
    K = d.n_active
    moe.set_flags(M.MHIP_DECODE_FORCE_ABORT)
    try:
        x0 = oracle.synth_x(W.X_SEED + 31, 1, d.dim)
        x = x0.copy()
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        rc = M.lib().mia_moe_layer_ex(moe.h, 2, x.ctypes.data, 1, None, idx.ctypes.data,
                                      w.ctypes.data, None)
        assert rc == 0, M.lib().mia_moe_error(moe.h).decode()
        assert moe.decode_status()[0] == 4, "the decode launch was not the aborted one"
        xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, 2, x0[0])
        assert np.array_equal(idx, io[0])
        assert np.array_equal(w.view(np.uint32), wo[0].view(np.uint32))
        assert np.array_equal(x[0].view(np.uint32), xo[0].view(np.uint32))

        xg, ig, wg = moe.decode(0, 3, x0[0])
        assert moe.decode_status()[0] == 4
        x = x0[0]
        for l in range(3):
            xo, io, wo, _, _ = run_oracle_layer(oracle, moe, d, l, x)
            assert np.array_equal(ig[l], io[0]), "layer %d indices" % l
            assert np.array_equal(wg[l].view(np.uint32), wo[0].view(np.uint32)), "layer %d w" % l
            x = xo[0]
        assert np.array_equal(xg.view(np.uint32), x.view(np.uint32))
    finally:
        moe.set_flags(0)
    xg, _, _ = moe.decode(0, 1, x0[0])  # the next launch runs normally
    assert moe.decode_status()[0] == 0


def test_decode_rejects_more_than_256_layers(qwen_dims, moe):
    say("test_decode_rejects_more_than_256_layers")
    L = M.lib()
    lay = M.Layout()
    assert L.mhip_layout_of(ctypes.byref(moe.dims), ctypes.byref(lay)) == 0
    rc = L.mhip_decode_stack(moe.gpu, ctypes.byref(moe.dims), ctypes.byref(lay), None, None,
                             None, None, None, None, M.DECODE_MAX_LAYERS + 1, None, None, None, 0)
    assert rc == -1
    assert b"outside [0, 256]" in L.mhip_error(moe.gpu)
