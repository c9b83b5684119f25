"""Full-depth GPU parity: the three 48-layer MoE-only stacks of the benchmark
workloads (src/model/forward.c:210-213 without the attention call) against
the oracle, on one 48-layer handle whose every layer has its own non-unit
ffn_norm (1 + 0.1 N(0, 1)), so the norm weight, its per-layer offset and the
decode kernel's prefetch of the next layer's norm are all exercised.

- decode48 (one token, the persistent decode kernel, exact router: the
  default): teacher-forced, one launch per layer on the oracle's own input,
  every layer bit-equal; then one free-running 48-layer launch from x0,
  through the device-pointer entry (mia_moe_decode_dev) and the host entry
  (mia_moe_decode), bit-equal to the oracle's free-running 48-layer chain
  from the same x0 (routing, gate weights and output of every layer), on two
  seeds. With MHIP_DECODE_CERTIFIED (gate weights from the parallel logits)
  a 48-layer launch is audited on its own trajectory: every layer routed as
  the oracle routes that layer's input, every update within TOL.
- batch64x48 (64 tokens, the vector kernels): every layer bit-equal to the
  oracle, each on the previous layer's output, and the one-call 48-layer
  stack bit-equal to the oracle's stack.
- prefill4096x48 (4096 tokens, the matrix-core kernels): each layer on the
  GPU's own previous output; every token's logits, expert indices, gate
  weights and layer output bit-equal to the oracle's at every layer.

TOL: max|diff| / max|ref| <= 1e-3 (tools/e2e/e2e_test.go:101-107), on the
update x_out - x_in and on x_out.
"""
import os
import sys

import numpy as np
import pytest

import motoria_amd as M
from motoria_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-3
L = 48
NTHREADS = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def layer_norm(layer, dim):
    rng = np.random.default_rng(1000 + layer)
    return (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)


@pytest.fixture(scope="module")
def deep(oracle, qwen_dims):
    d = qwen_dims
    say("open 48-layer handle (max_tokens 4096), distinct non-unit ffn_norm per layer")
    m = M.Moe(n_layers=L, max_tokens=4096, device=0, **W.SHAPE)
    m.synth(W.WEIGHT_SEED)
    norms = [layer_norm(l, d.dim) for l in range(L)]
    routers = [oracle.synth_router(W.WEIGHT_SEED, l, d) for l in range(L)]
    for l in range(L):
        m.set_layer(l, norms[l], routers[l])
    m.sync()
    yield m, norms, routers
    m.close()


def blobs_of(moe, d, layer, need):
    out = [None] * d.n_experts
    for e in sorted(set(int(v) for v in np.asarray(need).ravel())):
        out[e] = moe.read_expert(layer, e)
    return out


def oracle_layer(O, d, moe, norms, routers, layer, x, bucketed=False):
    """The oracle's layer on x[T][dim] with the experts read back from HBM
    (only those its own routing selects)."""
    x = np.array(x, np.float32, ndmin=2)
    idx, _, _ = O.route_tokens(d, x, norms[layer], routers[layer], nthreads=NTHREADS)
    blobs = blobs_of(moe, d, layer, idx)
    if bucketed:
        xo, io, wo, lo = O.moe_layer_bucketed(d, x, norms[layer], routers[layer], blobs,
                                              nthreads=NTHREADS)
    else:
        xo, io, wo, lo, _ = O.moe_layer(d, x, norms[layer], routers[layer], blobs,
                                        nthreads=NTHREADS)
    assert np.array_equal(io, idx)
    return xo, io, wo, lo


# ---- decode48 ---------------------------------------------------------------------

def test_decode48_teacher_forced(oracle, qwen_dims, deep):
    say("test_decode48_teacher_forced")
    moe, norms, routers = deep
    d = qwen_dims
    x = oracle.synth_x(W.X_SEED, 1, d.dim)[0]
    for l in range(L):
        xo, io, wo, _ = oracle_layer(oracle, d, moe, norms, routers, l, x)
        xg, ig, wg = moe.decode(l, l + 1, x)
        st = moe.decode_status()
        assert st[0] == 0, "layer %d: decode aborted %s" % (l, st)
        assert np.array_equal(ig[0], io[0]), "layer %d: idx %s vs %s" % (l, ig[0], io[0])
        assert np.array_equal(bits(wg[0]), bits(wo[0])), "layer %d: gate weights" % l
        assert np.array_equal(bits(xg), bits(xo[0])), \
            "layer %d: output rel err %.2e" % (l, rel(xg - x, xo[0] - x))
        x = xo[0]
        if l % 12 == 11:
            say("  layers 0..%d: bit-equal" % l)


def oracle_chain(oracle, d, moe, norms, routers, x0):
    """The oracle's free-running chain of the 48 layers from x0 (forward.c:
    210-213 without the attention): every layer's input, indices and gate
    weights."""
    xs, ids, ws = [np.asarray(x0, np.float32)], [], []
    for l in range(L):
        xo, io, wo, _ = oracle_layer(oracle, d, moe, norms, routers, l, xs[-1])
        xs.append(xo[0])
        ids.append(io[0])
        ws.append(wo[0])
    return xs, np.array(ids), np.array(ws)


@pytest.mark.parametrize("seed_off", [5, 6])
def test_decode48_one_launch_equals_oracle_chain(oracle, qwen_dims, deep, seed_off):
    """One 48-layer launch from x0 reproduces the oracle's free-running
    48-layer chain bit for bit: through mia_moe_decode_dev on device memory
    (the launch the benchmark times) and through the host entry
    mia_moe_decode (its indices and gate weights of every layer too)."""
    seed = W.X_SEED + seed_off
    say("test_decode48_one_launch_equals_oracle_chain seed %d" % seed)
    moe, norms, routers = deep
    d = qwen_dims
    x0 = oracle.synth_x(seed, 1, d.dim)[0]
    xs, ids, ws = oracle_chain(oracle, d, moe, norms, routers, x0)
    # the device-pointer entry
    d_x = moe.malloc(d.dim * 4)
    try:
        moe.h2d(d_x, x0)
        moe.decode_dev(0, L, d_x)
        moe.sync()
        st = moe.decode_status()
        xd = moe.d2h(d_x, d.dim, np.float32)
    finally:
        moe.free(d_x)
    assert st[0] == 0, "decode aborted %s" % st
    assert np.array_equal(bits(xd), bits(xs[L])), \
        "mia_moe_decode_dev: 48-layer output rel err %.2e" % rel(xd, xs[L])
    # the host entry, with the routing of every layer
    xg, ig, wg = moe.decode(0, L, x0)
    assert moe.decode_status()[0] == 0
    for l in range(L):
        assert np.array_equal(ig[l], ids[l]), "layer %d: idx %s vs %s" % (l, ig[l], ids[l])
        assert np.array_equal(bits(wg[l]), bits(ws[l])), "layer %d: gate weights" % l
    assert np.array_equal(bits(xg), bits(xs[L])), \
        "mia_moe_decode: 48-layer output rel err %.2e" % rel(xg, xs[L])
    say("  seed %d: x, indices and gate weights of all 48 layers bit-equal to the oracle's "
        "chain (status %s)" % (seed, st))


def test_decode48_certified_audit(oracle, qwen_dims, deep):
    """MHIP_DECODE_CERTIFIED: one 48-layer launch from x0, audited layer by
    layer on its own trajectory. The input of layer l is the output of a
    launch of layers [0, l) from x0: every launch runs the same per-layer
    code, so its first l layers are the 48-layer launch's (checked: the
    prefix launch's routing of those layers equals the 48-layer launch's,
    and the 48-layer launch is repeated and compared bit for bit). At every
    layer the oracle, given that input, must route exactly as the launch did
    and produce the update within TOL. The oracle's free-running chain is
    reported beside it (it drifts: the parallel gate weights differ by ~1e-6,
    which flips Q8 codes over 48 layers)."""
    say("test_decode48_certified_audit")
    moe, norms, routers = deep
    d = qwen_dims
    moe.set_flags(M.MHIP_DECODE_CERTIFIED)
    try:
        x0 = oracle.synth_x(W.X_SEED + 5, 1, d.dim)[0]
        xg, ig, _ = moe.decode(0, L, x0)
        assert moe.decode_status()[0] == 0
        xg2, ig2, _ = moe.decode(0, L, x0)
        assert np.array_equal(bits(xg), bits(xg2)) and np.array_equal(ig, ig2), \
            "not deterministic"
        xin = [x0]
        for l in range(1, L):
            xp, ip, _ = moe.decode(0, l, x0)
            assert np.array_equal(ip, ig[:l]), "prefix launch [0, %d) routed differently" % l
            xin.append(xp)
        xin.append(xg)
    finally:
        moe.set_flags(0)
    worst = 0.0
    for l in range(L):
        xo, io, _, _ = oracle_layer(oracle, d, moe, norms, routers, l, xin[l])
        assert np.array_equal(ig[l], io[0]), "layer %d: routing of the launch's own input" % l
        e = rel(xin[l + 1] - xin[l], xo[0] - xin[l])
        worst = max(worst, e)
        assert e <= TOL, "layer %d: update rel err %.2e" % (l, e)
    xs, _, _ = oracle_chain(oracle, d, moe, norms, routers, x0)
    say("  every layer of the certified launch routed as the oracle routes its input, worst "
        "update rel err %.2e; the oracle's free-running chain ends %.2e (relative) away"
        % (worst, rel(xg, xs[L])))


# ---- batch64x48 -------------------------------------------------------------------

def test_batch64x48_bit_exact(oracle, qwen_dims, deep):
    say("test_batch64x48_bit_exact")
    moe, norms, routers = deep
    d = qwen_dims
    x0 = oracle.synth_x(W.X_SEED, 64, d.dim)
    xs = moe.stack(0, L, x0)  # one call, 48 layers
    x = x0
    for l in range(L):
        xg, ig, wg, lg = moe.layer(l, x)
        xo, io, wo, lo = oracle_layer(oracle, d, moe, norms, routers, l, x)
        assert np.array_equal(ig, io), "layer %d indices" % l
        assert np.array_equal(bits(lg), bits(lo)), "layer %d logits" % l
        assert np.array_equal(bits(wg), bits(wo)), "layer %d gate weights" % l
        assert np.array_equal(bits(xg), bits(xo)), \
            "layer %d output: rel err %.2e" % (l, rel(xg - x, xo - x))
        x = xo
        if l % 12 == 11:
            say("  layers 0..%d bit-equal (%d experts touched at layer %d)"
                % (l, len(set(ig.ravel().tolist())), l))
    assert np.array_equal(bits(xs), bits(x)), "48-layer stack call differs from the oracle"


# ---- prefill4096x48 ---------------------------------------------------------------

@pytest.fixture(scope="module")
def prefill_chain(oracle, qwen_dims, deep):
    """The GPU's own 48-layer chain at T = 4096: x before every layer and the
    routing every layer produced."""
    moe, _, _ = deep
    say("prefill4096x48: GPU chain, one layer call per layer")
    x = oracle.synth_x(W.X_SEED + 11, 4096, qwen_dims.dim)
    xs, routing = [x], []
    for l in range(L):
        xg, ig, wg, lg = moe.layer(l, xs[-1])
        xs.append(xg)
        routing.append((ig, wg, lg))
    return xs, routing


@pytest.mark.parametrize("group", range(4))
def test_prefill4096x48_every_token(oracle, qwen_dims, deep, prefill_chain, group):
    say("test_prefill4096x48_every_token layers %d..%d" % (12 * group, 12 * group + 11))
    moe, norms, routers = deep
    d = qwen_dims
    xs, routing = prefill_chain
    for l in range(12 * group, 12 * group + 12):
        x = xs[l]
        ig, wg, lg = routing[l]
        xo, io, wo, lo = oracle_layer(oracle, d, moe, norms, routers, l, x, bucketed=True)
        assert np.array_equal(bits(lg), bits(lo)), "layer %d logits" % l
        assert np.array_equal(ig, io), "layer %d expert indices" % l
        assert np.array_equal(bits(wg), bits(wo)), "layer %d gate weights" % l
        assert np.array_equal(bits(xs[l + 1]), bits(xo)), "layer %d output" % l
    say("  4096 tokens x 12 layers: routing and outputs bit-equal")
