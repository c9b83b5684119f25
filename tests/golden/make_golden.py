"""Writes the golden vectors of tests/golden/ from the reference's own code.

Run in the container that holds the reference sources, after
`make -C oracle ref` (which compiles src/tensor/quant.c, src/tensor/matmul.c,
src/storage/expert_cache.c and, through oracle/ref_shim.c, the static moe()
of src/model/forward.c into oracle/_ref/libmia_ref.so):

    python tests/golden/make_golden.py

Inputs are regenerated from seeds (the reference tests' xorshift generator,
tests/check.h:37-44, and include/mia/synth.h); the fixtures hold the inputs'
seeds and hashes and the reference's outputs as raw bits.
"""
import hashlib
import json
import os
import platform
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402


def xorshift_uniform(n, state=0x9E3779B9):
    """tests/check.h:37-44 of the reference: [-1, 1) floats."""
    out = np.zeros(n, dtype=np.float32)
    g = state
    for i in range(n):
        g ^= (g << 13) & 0xFFFFFFFF
        g ^= g >> 17
        g ^= (g << 5) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(g & 0xFFFFFF) / np.float32(0x1000000) * np.float32(2.0)
                            - np.float32(1.0))
    return out, g


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref_quantize(R, x):
    out = np.zeros(x.size // 32 * 36, np.uint8)
    R.mia_quantize_row_q8(x.ctypes.data, out.ctypes.data, x.size)
    return out


def ref_matvec(R, w, t, x, rows, cols):
    out = np.zeros(rows, np.float32)
    xq = np.zeros(max(cols // 32, 1) * 36, np.uint8)
    R.mia_matvec_scalar(out.ctypes.data, w.ctypes.data, t, x.ctypes.data, xq.ctypes.data, rows,
                        cols)
    return out


def main():
    R = O.ref()
    fixtures = {}

    # Q8_0 quantization of xorshift rows (tests/test_quant.c:10-22 draws x*3).
    u, _ = xorshift_uniform(4096)
    x = (u * np.float32(3.0)).astype(np.float32)
    fixtures["quant"] = dict(x_sha=np.frombuffer(bytes.fromhex(sha(x)), np.uint8),
                             q=ref_quantize(R, x))

    # mat-vec at the reference tests' shapes (tests/test_matmul.c:31-49).
    u, _ = xorshift_uniform(2048 * 768 + 768)
    for rows, cols in [(7, 32), (1024, 512)]:
        w = u[: rows * cols].copy()
        xv = u[rows * cols: rows * cols + cols].copy()
        fixtures["matvec_f32_%dx%d" % (rows, cols)] = dict(
            w_sha=np.frombuffer(bytes.fromhex(sha(w)), np.uint8),
            x_sha=np.frombuffer(bytes.fromhex(sha(xv)), np.uint8),
            out=ref_matvec(R, w, 0, xv, rows, cols))
    for rows, cols in [(5, 64), (2048, 768)]:
        w = u[: rows * cols].copy()
        xv = u[rows * cols: rows * cols + cols].copy()
        wq = np.concatenate([ref_quantize(R, w[r * cols:(r + 1) * cols]) for r in range(rows)])
        fixtures["matvec_q8_%dx%d" % (rows, cols)] = dict(
            w_sha=np.frombuffer(bytes.fromhex(sha(wq)), np.uint8),
            x_sha=np.frombuffer(bytes.fromhex(sha(xv)), np.uint8),
            out=ref_matvec(R, wq, 1, xv, rows, cols))

    # Whole layers through the reference's moe().
    layers = [
        ("layer_tiny", O.TINY, 5, 11, 32),
        ("layer_qwen_decode", O.QWEN3_30B_A3B, 42, 43, 4),
    ]
    meta_layers = {}
    for name, shape, wseed, xseed, T in layers:
        d = O.dims(**shape)
        xin = O.synth_x(xseed, T, d.dim)
        router = O.synth_router(wseed, 0, d)
        norm = np.ones(d.dim, np.float32)
        blobs = [O.synth_expert_blob(wseed, 0, e, d) for e in range(d.n_experts)]
        xo, idx_loaded, idx, w, logits, xn = O.ref_moe_layer(d, xin, norm, router, blobs)
        assert np.array_equal(idx_loaded, idx)
        used = sorted(set(idx.ravel().tolist()))
        fixtures[name] = dict(x_in_sha=np.frombuffer(bytes.fromhex(sha(xin)), np.uint8),
                              x_out=xo, idx=idx, w=w, logits=logits, xn=xn,
                              used=np.array(used, np.int32),
                              blob_sha=np.stack([np.frombuffer(bytes.fromhex(sha(blobs[e])),
                                                               np.uint8) for e in used]))
        meta_layers[name] = dict(shape=shape, weight_seed=wseed, x_seed=xseed, tokens=T,
                                 layer=0)

    for name, arrs in fixtures.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)
    glibc = " ".join(platform.libc_ver())
    cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.split("\n")[0]
    manifest = dict(
        generator="tests/golden/make_golden.py",
        reference_build="oracle/Makefile target ref: gcc -std=c99 -O3 -ffp-contract=off of "
                        "src/tensor/quant.c, src/tensor/matmul.c, src/storage/expert_cache.c "
                        "and src/model/forward.c (via oracle/ref_shim.c)",
        libc=glibc, compiler=cc, cpu=platform.processor() or platform.machine(),
        layers=meta_layers, files=sorted(n + ".npz" for n in fixtures))
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print("wrote", len(fixtures), "fixtures")


if __name__ == "__main__":
    main()
