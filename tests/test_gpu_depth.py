"""Full-depth GPU parity: the three 48-layer MoE-only stacks of the benchmark
workloads (src/model/forward.c:210-213 without the attention call) against
the oracle, on one 48-layer handle whose every layer has its own non-unit
ffn_norm (1 + 0.1 N(0, 1)), so the norm weight, its per-layer offset and the
decode kernel's prefetch of the next layer's norm are all exercised.

- decode48 (one token, the persistent decode kernel): teacher-forced, one
  launch per layer on the oracle's own input, expert indices bit-equal and
  the update within TOL; then one 48-layer launch compared end to end, where
  a routing difference may only start at a near-tie of the oracle's gate
  probabilities (the two paths' inputs differ by rounding there).
- batch64x48 (64 tokens, the vector kernels): every layer bit-equal to the
  oracle, each on the previous layer's output, and the one-call 48-layer
  stack bit-equal to the oracle's stack.
- prefill4096x48 (4096 tokens, the matrix-core kernels): each layer on the
  GPU's own previous output; every token's logits, expert indices and gate
  weights bit-equal to the oracle's at every layer, and the layer outputs of
  all 4096 tokens within TOL at every layer.

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
NEAR_TIE = 1e-4  # relative gap of the oracle's probabilities that rounding of the input can cross


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
    worst = 0.0
    for l in range(L):
        xo, io, wo, _ = oracle_layer(oracle, d, moe, norms, routers, l, x)
        xg, ig, wg = moe.decode(l, l + 1, x)
        st = moe.decode_status()
        assert st[0] == 0, "layer %d: decode aborted %s" % (l, st)
        assert np.array_equal(ig[0], io[0]), "layer %d: idx %s vs %s" % (l, ig[0], io[0])
        e = rel(xg - x, xo[0] - x)
        worst = max(worst, e)
        assert e <= TOL and rel(wg[0], wo[0]) <= TOL, "layer %d: rel err %.2e" % (l, e)
        x = xo[0]
        if l % 12 == 11:
            say("  layers 0..%d: indices bit-equal, worst update rel err %.2e" % (l, worst))


def test_decode48_one_launch_divergence_audit(oracle, qwen_dims, deep):
    say("test_decode48_one_launch_divergence_audit")
    moe, norms, routers = deep
    d = qwen_dims
    K = d.n_active
    for seed in (W.X_SEED + 5, W.X_SEED + 6):
        x0 = oracle.synth_x(seed, 1, d.dim)[0]
        xg, ig, _ = moe.decode(0, L, x0)
        st = moe.decode_status()
        assert st[0] == 0, st
        x = x0
        diverged = None
        for l in range(L):
            xo, io, _, lo = oracle_layer(oracle, d, moe, norms, routers, l, x)
            if not np.array_equal(ig[l], io[0]):
                diverged = l
                # the oracle's gate probabilities at this layer: every expert
                # that differs must sit at a near-tie of the ordering
                p = oracle.softmax(lo[0])
                top = np.sort(p)[::-1]
                kth = top[K - 1]
                for e in set(ig[l].tolist()) ^ set(io[0].tolist()):
                    assert abs(p[e] - kth) <= NEAR_TIE * kth, \
                        "layer %d: expert %d differs away from a near-tie" % (l, e)
                if set(ig[l].tolist()) == set(io[0].tolist()):
                    # same set, different order: the swapped pair is a near-tie
                    for j in range(K):
                        if ig[l][j] != io[0][j]:
                            a, b = p[ig[l][j]], p[io[0][j]]
                            assert abs(a - b) <= NEAR_TIE * max(a, b), "layer %d order" % l
                break
            x = xo[0]
        if diverged is None:
            e = rel(xg - x0, x - x0)
            say("  seed %d: 48 layers routed identically, end-to-end update rel err %.2e"
                % (seed, e))
            assert e <= TOL and rel(xg, x) <= TOL
        else:
            say("  seed %d: routing first differs at layer %d, at a near-tie" % (seed, diverged))


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
    worst = 0.0
    for l in range(12 * group, 12 * group + 12):
        x = xs[l]
        ig, wg, lg = routing[l]
        xo, io, wo, lo = oracle_layer(oracle, d, moe, norms, routers, l, x, bucketed=True)
        assert np.array_equal(bits(lg), bits(lo)), "layer %d logits" % l
        assert np.array_equal(ig, io), "layer %d expert indices" % l
        assert np.array_equal(bits(wg), bits(wo)), "layer %d gate weights" % l
        e_up, e_out = rel(xs[l + 1] - x, xo - x), rel(xs[l + 1], xo)
        worst = max(worst, e_up)
        assert e_up <= TOL and e_out <= TOL, "layer %d: rel err %.2e / %.2e" % (l, e_up, e_out)
    say("  4096 tokens x 12 layers: routing bit-equal, worst update rel err %.2e" % worst)
