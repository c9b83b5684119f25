"""The C-ABI library loads and exports every function include/ declares
(no compute calls: this runs without a GPU)."""
import ctypes
import os
import re
import subprocess

import motoria_amd as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = ["include/mia_hip.h", "include/mia/quant.h", "include/mia/matmul.h",
           "include/mia/matvec_cache.h", "include/mia/moe.h", "include/mia/model_gpu.h",
           "include/mia/serve.h", "include/mia/tensor_error.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(os.path.join(ROOT, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(([^;{}]*)\)\s*;", text):
            names.add(m.group(1))
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", M.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_loads():
    L = M.lib()
    assert isinstance(L, ctypes.CDLL)


def test_every_declared_function_is_exported_and_bound():
    declared = declared_functions()
    assert len(declared) > 40
    exported = exported_symbols()
    missing = sorted(declared - exported)
    assert not missing, "declared in include/ but not exported: %s" % missing
    unbound = sorted(declared - set(M.SIGNATURES))
    assert not unbound, "not bound in motoria_amd.SIGNATURES: %s" % unbound
    extra = sorted(set(M.SIGNATURES) - declared)
    assert not extra, "bound but not declared: %s" % extra


def test_row_bytes_by_type():
    # tests/test_quant.c:4-8 of the reference (pure arithmetic, no GPU call)
    L = M.lib()
    assert L.mia_row_bytes(0, 64) == 256
    assert L.mia_row_bytes(1, 64) == 72
    assert L.mia_row_bytes(1, 2048) == 2304 and L.mia_row_bytes(1, 768) == 864


def test_layout_matches_blob_size():
    d = M.Dims(2048, 128, 8, 768, 1, 1e-6)
    lay = M.Layout()
    assert M.lib().mhip_layout_of(ctypes.byref(d), ctypes.byref(lay)) == 0
    # Regrouping keeps 1.125 bytes per weight (the .mia blob size exactly, up
    # to the start of the block-major scale copy), plus that copy.
    assert lay.gate_st == 5308416
    scales = 2 * 768 * 64 * 4 + 2048 * 24 * 4
    assert lay.expert_bytes == 5308416 + scales
    for off in (lay.gate_q, lay.up_q, lay.down_q, lay.gate_s, lay.up_s, lay.down_s,
                lay.gate_st, lay.up_st, lay.down_st):
        assert off % 256 == 0


def test_layout_rejects_unsupported_shapes():
    lay = M.Layout()
    for bad in [M.Dims(2047, 128, 8, 768, 1, 1e-6), M.Dims(2048, 300, 8, 768, 1, 1e-6),
                M.Dims(2048, 128, 65, 768, 1, 1e-6), M.Dims(2048, 4, 8, 768, 1, 1e-6)]:
        assert M.lib().mhip_layout_of(ctypes.byref(bad), ctypes.byref(lay)) == -1


def test_no_oracle_in_product():
    """The product library links nothing from oracle/ and exports no oracle
    symbol; the package never imports the oracle."""
    exported = exported_symbols()
    assert not any(s.startswith("orc_") or s.startswith("ref_") for s in exported)
    deps = subprocess.run(["ldd", M.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in deps
    for dirpath, _, files in os.walk(os.path.join(ROOT, "motoria_amd")):
        for f in files:
            if f.endswith((".py", ".c", ".h", ".hip")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "mia_oracle" not in text, f


def test_decode_stack_rejects_more_than_256_layers_before_any_device_call():
    """Exchange tags hold the layer in 8 bits: one decode launch covers at
    most 256 layers, and the argument check comes before any device call (so
    it runs here without a GPU and without a context)."""
    d = M.Dims(2048, 128, 8, 768, 1, 1e-6)
    lay = M.Layout()
    L = M.lib()
    assert L.mhip_layout_of(ctypes.byref(d), ctypes.byref(lay)) == 0
    for bad in (M.DECODE_MAX_LAYERS + 1, 1000, -1):
        rc = L.mhip_decode_stack(None, ctypes.byref(d), ctypes.byref(lay), None, None, None,
                                 None, None, None, bad, None, None, None, 0)
        assert rc == -1


def test_python_constants_match_the_headers():
    """Every MHIP_* constant the Python bindings mirror has the header's value
    (and the decode trace's window, TRACE_L0 / TRACE_NL / TRACE_SLOTS)."""
    defines = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, h)).read(), flags=re.S)
        for m in re.finditer(r"^#define\s+(MHIP_\w+)\s+(\d+)\s*$", text, flags=re.M):
            defines[m.group(1)] = int(m.group(2))
    mirrored = [k for k in defines if hasattr(M, k)]
    assert len(mirrored) > 10
    for k in mirrored:
        assert getattr(M, k) == defines[k], k
    assert (M.TRACE_L0, M.TRACE_NL, M.TRACE_SLOTS) == (
        defines["MHIP_TRACE_L0"], defines["MHIP_TRACE_NL"], defines["MHIP_TRACE_SLOTS"])


def test_tensor_ops_report_a_missing_gpu():
    """The reference's void tensor ops (mia_matvec, mia_quantize_row_q8,
    mia_dequantize_row) cannot return an error: without a GPU they fill their
    outputs with NaN and mia_tensor_error reports the failure once (reading
    it clears it). Runs only where no GPU is visible (the error path)."""
    import numpy as np
    import pytest

    L = M.lib()
    if L.mhip_device_count() > 0:
        pytest.skip("a GPU is visible: the failure path is not reachable")
    L.mia_tensor_error()
    out = np.zeros(4, np.float32)
    w = np.ones((4, 32), np.float32)
    x = np.ones(32, np.float32)
    L.mia_matvec(out.ctypes.data, w.ctypes.data, 0, x.ctypes.data, None, 4, 32)
    assert np.all(np.isnan(out))
    y = np.zeros(4 * 36, np.uint8)
    L.mia_quantize_row_q8(np.ones(128, np.float32).ctypes.data, y.ctypes.data, 128)
    assert np.all(np.isnan(y.view(np.float32).reshape(4, 9)[:, 0]))
    msg = L.mia_tensor_error()
    assert msg is not None and b"cannot open a GPU" in msg and b"more failures" in msg
    assert L.mia_tensor_error() is None


def test_tensor_ops_can_abort_instead():
    """With MIA_ABORT_ON_GPU_ERROR set, a failing tensor op aborts the
    process with its message (the reference engine's own behaviour on an
    unrecoverable error). Runs only where no GPU is visible."""
    import sys

    import pytest

    if M.lib().mhip_device_count() > 0:
        pytest.skip("a GPU is visible: the failure path is not reachable")
    code = ("import numpy as np, motoria_amd as M; o = np.zeros(4, np.float32); "
            "w = np.ones((4, 32), np.float32); x = np.ones(32, np.float32); "
            "M.lib().mia_matvec(o.ctypes.data, w.ctypes.data, 0, x.ctypes.data, None, 4, 32)")
    env = dict(os.environ, MIA_ABORT_ON_GPU_ERROR="1", PYTHONPATH=ROOT)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0 and "cannot open a GPU" in r.stderr
