"""The allocation-free decode entry point, mhip_decode_stack_noalloc, against
the workspace entry point mhip_decode_stack on the same inputs: x, routing
and status bit-equal, on two calls in a row, the second with fewer layers
(a smaller input), on a 4-layer synthetic table with non-unit ffn_norm.
Both entry points run the same kernel, whose results do not depend on the
workspace it exchanges through."""
import ctypes
import sys

import numpy as np
import pytest

import motoria_amd as M
from motoria_amd import workloads as W

pytestmark = pytest.mark.gpu

NL = 4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Stack:
    """A synthetic NL-layer decode stack in device memory of context g."""

    def __init__(self, g):
        L = M.lib()
        self.g = g
        self.dims = M.Dims(**W.SHAPE)
        self.lay = M.Layout()
        assert L.mhip_layout_of(ctypes.byref(self.dims), ctypes.byref(self.lay)) == 0
        d, E = self.dims.dim, self.dims.n_experts
        self.table = g.malloc(NL * E * self.lay.expert_bytes)
        g.check(L.mhip_table_synth(g.h, ctypes.byref(self.dims), self.table, W.WEIGHT_SEED, 0,
                                   NL), "table synth")
        self.rt = g.malloc(NL * d * E * 4)
        self.rdl = g.malloc(NL * d * E * 4)
        for l in range(NL):
            g.check(L.mhip_router_synth(g.h, ctypes.byref(self.dims), self.rt + l * d * E * 4,
                                        self.rdl + l * d * E * 4, W.WEIGHT_SEED, l),
                    "router synth")
        norms = np.concatenate([
            (1.0 + 0.1 * np.random.default_rng(50 + l).standard_normal(d)).astype(np.float32)
            for l in range(NL)])
        self.norm = g.upload(norms)
        self.ws = g.malloc(L.mhip_decode_ws_bytes())

    def run(self, noalloc, nl, x, g=None):
        """One token through layers [0, nl): (x, idx, w, status)."""
        g = g or self.g
        L = M.lib()
        K = self.dims.n_active
        dx = g.upload(np.ascontiguousarray(x, np.float32))
        didx = g.malloc(nl * K * 4)
        dw = g.malloc(nl * K * 4)
        args = (ctypes.byref(self.dims), ctypes.byref(self.lay), self.table, self.rdl, self.rt,
                self.norm, None, dx, nl)
        if noalloc:
            dst = g.malloc(16)
            g.check(L.mhip_decode_stack_noalloc(g.h, *args, didx, dw, dst, 0), "noalloc")
            g.check(L.mhip_sync(g.h), "sync")
            st = g.download(dst, 4, np.int32)
            g.free(dst)
        else:
            g.check(L.mhip_decode_stack(g.h, *args, self.ws, didx, dw, 0), "decode stack")
            st4 = (ctypes.c_int * 4)()
            g.check(L.mhip_decode_status(g.h, self.ws, st4), "status")
            st = np.array(list(st4), np.int32)
        out = (g.download(dx, x.size, np.float32), g.download(didx, (nl, K), np.int32),
               g.download(dw, (nl, K), np.float32), st)
        for p in (dx, didx, dw):
            g.free(p)
        return out


@pytest.fixture(scope="module")
def stack():
    g = M.Gpu(0)
    st = Stack(g)
    yield st
    g.close()


def _same(a, b, what):
    for u, v, name in zip(a, b, ("x", "idx", "w", "status")):
        u, v = np.asarray(u), np.asarray(v)
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), "%s: %s differs" % (what, name)


def test_noalloc_decode_matches_workspace_entry_point(oracle, stack):
    say("test_noalloc_decode_matches_workspace_entry_point")
    for nl, seed in ((NL, W.X_SEED + 40), (2, W.X_SEED + 41)):  # second call: smaller input
        x = oracle.synth_x(seed, 1, 2048)[0]
        ref = stack.run(False, nl, x)
        got = stack.run(True, nl, x)
        assert ref[3][0] == 0 and got[3][0] == 0, (ref[3], got[3])
        _same(ref, got, "%d layers" % nl)
        say("  %d layers: bit-equal, status %s" % (nl, got[3].tolist()))


def test_noalloc_decode_shared_by_contexts_of_one_device(oracle, stack):
    """A second context on the same GPU uses the same workspace (its
    launches continue the device's count), and results stay bit-equal."""
    say("test_noalloc_decode_shared_by_contexts_of_one_device")
    x = oracle.synth_x(W.X_SEED + 42, 1, 2048)[0]
    ref = stack.run(False, 3, x)
    g2 = M.Gpu(0)
    try:
        a = stack.run(True, 3, x, g=g2)
        b = stack.run(True, 3, x)
    finally:
        g2.close()
    _same(ref, a, "second context")
    _same(ref, b, "first context after the second")


def test_noalloc_decode_ordered_across_streams(oracle, stack):
    """Two contexts (two streams) of one GPU queue calls back to back with
    no host wait between them: the second call waits for the first launch
    (an event on the shared workspace), so both results equal the workspace
    entry point's."""
    say("test_noalloc_decode_ordered_across_streams")
    L = M.lib()
    K = stack.dims.n_active
    xs = [oracle.synth_x(W.X_SEED + 43 + i, 1, 2048)[0] for i in range(2)]
    refs = [stack.run(False, NL, x) for x in xs]
    g2 = M.Gpu(0)
    try:
        ctxs = [stack.g, g2]
        bufs = []
        for g, x in zip(ctxs, xs):
            bufs.append((g.upload(np.ascontiguousarray(x, np.float32)), g.malloc(NL * K * 4),
                         g.malloc(NL * K * 4), g.malloc(16)))
        for g, (dx, didx, dw, dst) in zip(ctxs, bufs):
            g.check(L.mhip_decode_stack_noalloc(
                g.h, ctypes.byref(stack.dims), ctypes.byref(stack.lay), stack.table, stack.rdl,
                stack.rt, stack.norm, None, dx, NL, didx, dw, dst, 0), "noalloc")
        for g in ctxs:
            g.check(L.mhip_sync(g.h), "sync")
        for i, (g, (dx, didx, dw, dst)) in enumerate(zip(ctxs, bufs)):
            got = (g.download(dx, 2048, np.float32), g.download(didx, (NL, K), np.int32),
                   g.download(dw, (NL, K), np.float32), g.download(dst, 4, np.int32))
            assert got[3][0] == 0, got[3]
            _same(refs[i], got, "stream %d" % i)
            for p in (dx, didx, dw, dst):
                g.free(p)
    finally:
        g2.close()


def test_noalloc_decode_rejects_more_than_256_layers(stack):
    say("test_noalloc_decode_rejects_more_than_256_layers")
    L = M.lib()
    g = stack.g
    rc = L.mhip_decode_stack_noalloc(g.h, ctypes.byref(stack.dims), ctypes.byref(stack.lay),
                                     stack.table, stack.rdl, stack.rt, stack.norm, None, None,
                                     M.DECODE_MAX_LAYERS + 1, None, None, None, 0)
    assert rc == -1
    assert b"outside [0, 256]" in L.mhip_error(g.h)
