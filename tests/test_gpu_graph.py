"""The MoE stack as one HIP graph (mia_moe_stack_graph): every replay is
bit-equal to the eager stack (mia_moe_stack_dev) on the same input, with
eager work and device waits between the replays; the vector path (T = 64,
batched decode) and the matrix-core path (T = 300); a call with other
arguments records again."""
import sys

import numpy as np
import pytest

import motoria_amd as M
from motoria_amd import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("T,L", [(64, 6), (300, 3)])
def test_stack_graph_replays_bit_equal(T, L):
    say("test_stack_graph_replays_bit_equal T=%d L=%d" % (T, L))
    moe = M.Moe(n_layers=L, max_tokens=T, device=0, **W.SHAPE)
    try:
        moe.synth(W.WEIGHT_SEED)
        d = W.SHAPE["dim"]
        nbytes = T * d * 4
        d_x0, d_x, d_y = moe.malloc(nbytes), moe.malloc(nbytes), moe.malloc(nbytes)
        moe.synth_f32(d_x0, T * d, 77, 1 << 40, 1.0)
        copy = lambda dst: M.lib().mhip_d2d(moe.gpu, dst, d_x0, nbytes)  # noqa: E731
        copy(d_x)
        moe.stack_dev(0, L, d_x, T)
        want = moe.d2h(d_x, (T, d), np.float32)
        copy(d_x)
        moe.stack_dev(0, L - 1, d_x, T)
        want_short = moe.d2h(d_x, (T, d), np.float32)
        for r in range(4):
            copy(d_x)
            moe.stack_graph(0, L, d_x, T)
            moe.sync()
            got = moe.d2h(d_x, (T, d), np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "replay %d" % r
            # eager work between replays, on another buffer
            copy(d_y)
            moe.layer_dev(0, d_y, T)
            moe.sync()
        copy(d_x)
        moe.stack_graph(0, L - 1, d_x, T)  # other arguments: recorded again
        got = moe.d2h(d_x, (T, d), np.float32)
        assert np.array_equal(got.view(np.uint32), want_short.view(np.uint32))
        copy(d_x)
        moe.stack_graph(0, L - 1, d_x, T)
        got = moe.d2h(d_x, (T, d), np.float32)
        assert np.array_equal(got.view(np.uint32), want_short.view(np.uint32))
        say("  4 replays + re-recording bit-equal to the eager stack")
        for p in (d_x0, d_x, d_y):
            moe.free(p)
    finally:
        moe.close()
