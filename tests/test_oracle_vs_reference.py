"""The C restatement (oracle/) against the reference's own compiled code
(oracle/_ref, built from the reference sources by `make -C oracle ref`), bit
for bit, on inputs beyond the committed golden vectors. Skipped where the
reference build is absent (the GPU box has no reference sources)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")


def test_quantize_random_rows_bit_equal():
    R = O.ref()
    rng = np.random.default_rng(10)
    for scale in [1e-30, 1e-3, 1.0, 1e6]:
        x = (rng.normal(size=64 * 32) * scale).astype(np.float32)
        x[:32] = 0.0  # a zero block
        want = np.zeros(x.size // 32 * 36, np.uint8)
        R.mia_quantize_row_q8(x.ctypes.data, want.ctypes.data, x.size)
        assert np.array_equal(O.quantize_row_q8(x), want)


@pytest.mark.parametrize("rows,cols,wtype", [(64, 2048, 0), (128, 2048, 0), (768, 2048, 1),
                                             (2048, 768, 1), (3, 32, 1)])
def test_matvec_bit_equal(rows, cols, wtype):
    R = O.ref()
    rng = np.random.default_rng(rows + cols)
    w = (rng.normal(size=rows * cols) * 0.02).astype(np.float32)
    x = rng.normal(size=cols).astype(np.float32)
    if wtype == 1:
        w = np.concatenate([O.quantize_row_q8(w[r * cols:(r + 1) * cols]) for r in range(rows)])
    want = np.zeros(rows, np.float32)
    xq = np.zeros(max(cols // 32, 1) * 36, np.uint8)
    R.mia_matvec_scalar(want.ctypes.data, w.ctypes.data, wtype, x.ctypes.data, xq.ctypes.data,
                        rows, cols)
    assert np.array_equal(O.matvec(w, wtype, x, rows, cols).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("shape,T,seed", [("TINY", 64, 21), ("TINY", 64, 22),
                                          ("QWEN3_30B_A3B", 3, 23)])
def test_layer_bit_equal(shape, T, seed):
    d = O.dims(**getattr(O, shape))
    x = O.synth_x(seed + 100, T, d.dim)
    router = O.synth_router(seed, 0, d)
    norm = (1.0 + 0.1 * np.random.default_rng(seed).normal(size=d.dim)).astype(np.float32)
    blobs = [O.synth_expert_blob(seed, 0, e, d) for e in range(d.n_experts)]
    xo, idx, w, logits, xn = O.moe_layer(d, x, norm, router, blobs, nthreads=4)
    xr, il, ir, wr, lr, xnr = O.ref_moe_layer(d, x, norm, router, blobs)
    assert np.array_equal(idx, ir) and np.array_equal(il, ir)
    for a, b in [(xo, xr), (w, wr), (logits, lr), (xn, xnr)]:
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
