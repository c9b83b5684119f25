"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, never by the product package (motoria_amd).

`ref()` additionally loads oracle/_ref/libmia_ref.so, the reference's own
sources compiled by `make -C oracle ref` in the container that holds them.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

QK = 32
BLOCK_BYTES = 36

_i = ctypes.c_int
_f = ctypes.c_float
_p = ctypes.c_void_p
_u64 = ctypes.c_uint64


class Dims(ctypes.Structure):
    _fields_ = [("dim", _i), ("n_experts", _i), ("n_active", _i),
                ("expert_hidden", _i), ("norm_topk", _i), ("norm_eps", _f)]


QWEN3_30B_A3B = dict(dim=2048, n_experts=128, n_active=8, expert_hidden=768,
                     norm_topk=1, norm_eps=1e-6)
# The reference's tiny e2e model (tools/e2e/e2e_test.go:23-29).
TINY = dict(dim=64, n_experts=8, n_active=2, expert_hidden=32, norm_topk=1,
            norm_eps=1e-6)


def dims(**kw):
    return Dims(**kw)


def select(variant):
    """Which build the wrappers below call: "default" (oracle/liboracle.so,
    gcc -O3 -ffp-contract=off) or "native" (oracle/_native/liboracle.so, the
    same with -march=native, built by `make -C oracle native` on the host
    that runs it)."""
    global _LIB
    _LIB = None
    lib(variant)


class Sampler(ctypes.Structure):
    """orc_sampler (mia_oracle.h)."""
    _fields_ = [("temperature", _f), ("top_p", _f), ("n", _i), ("rng", _u64)]


class Model(ctypes.Structure):
    """orc_model (mia_oracle.h): the tensors of a whole model."""
    _fields_ = [("moe", Dims), ("n_layers", _i), ("n_heads", _i), ("n_kv_heads", _i),
                ("head_dim", _i), ("vocab", _i), ("wtype", _i), ("rope_theta", _f)] + [
        (n, _p) for n in ("token_embd", "output", "output_norm", "attn_norm", "q_norm",
                          "k_norm", "ffn_norm", "router", "wq", "wk", "wv", "wo", "blobs")]


def lib(variant=None):
    global _LIB
    if _LIB is None:
        name = os.path.join("_native", "liboracle.so") if variant == "native" else "liboracle.so"
        path = os.path.join(_HERE, name)
        if not os.path.exists(path):
            raise RuntimeError("oracle/%s is not built (make -C oracle%s)"
                               % (name, " native" if variant == "native" else ""))
        L = ctypes.CDLL(path)
        L.orc_row_bytes.restype = ctypes.c_size_t
        L.orc_row_bytes.argtypes = [_i, _i]
        L.orc_quantize_row_q8.argtypes = [_p, _p, _i]
        L.orc_dequantize_row.argtypes = [_i, _p, _p, _i]
        L.orc_matvec.argtypes = [_p, _p, _i, _p, _p, _i, _i]
        L.orc_rmsnorm.argtypes = [_p, _p, _p, _i, _f]
        L.orc_softmax.argtypes = [_p, _i]
        L.orc_top_k.argtypes = [_p, _i, _i, _p]
        L.orc_expf.restype = _f
        L.orc_expf.argtypes = [_f]
        for fn in ("orc_off_up", "orc_off_down", "orc_blob_bytes"):
            getattr(L, fn).restype = ctypes.c_size_t
            getattr(L, fn).argtypes = [ctypes.POINTER(Dims)]
        L.orc_moe_layer.argtypes = [ctypes.POINTER(Dims), _i, _p, _p, _p, _p, _p,
                                    _p, _p, _p, _p, _i]
        L.orc_moe_stack.argtypes = [ctypes.POINTER(Dims), _i, _i, _p, _p, _p, _p, _i]
        L.orc_moe_layer_bucketed.argtypes = [ctypes.POINTER(Dims), _i, _p, _p, _p, _p, _p,
                                             _p, _p, _p, _i]
        L.orc_model_step.argtypes = [ctypes.POINTER(Model), _p, _p, _i, _i, _i, _p, _p, _i]
        L.orc_rope_row.argtypes = [_p, _i, _i, _f]
        L.orc_sampler_init.argtypes = [ctypes.POINTER(Sampler), _f, _f, _i, _u64]
        L.orc_sampler_rand01.restype = _f
        L.orc_sampler_rand01.argtypes = [ctypes.POINTER(Sampler)]
        L.orc_sample.argtypes = [ctypes.POINTER(Sampler), _p]
        L.orc_route_tokens.argtypes = [ctypes.POINTER(Dims), _i, _p, _p, _p, _p, _p, _p, _p,
                                       _i]
        L.orc_route.argtypes = [_p, _i, _i, _i, _p, _p]
        L.orc_dispatch.argtypes = [_p, _i, _i, _i, _p, _p, _p, _p]
        L.orc_synth_x.argtypes = [_u64, _i, _i, _p]
        L.orc_synth_router.argtypes = [_u64, _i, ctypes.POINTER(Dims), _p]
        L.orc_synth_expert_blob.argtypes = [_u64, _i, _i, ctypes.POINTER(Dims), _p]
        _LIB = L
    return _LIB


def ref_available():
    return os.path.exists(os.path.join(_HERE, "_ref", "libmia_ref.so"))


def ref():
    """The reference build (its own quant.c/matmul.c/expert_cache.c/forward.c)."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libmia_ref.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/_ref is not built (make -C oracle ref)")
        R = ctypes.CDLL(path)
        R.mia_row_bytes.restype = ctypes.c_size_t
        R.mia_row_bytes.argtypes = [_i, _i]
        R.mia_quantize_row_q8.argtypes = [_p, _p, _i]
        R.mia_dequantize_row.argtypes = [_i, _p, _p, _i]
        R.mia_matvec.argtypes = [_p, _p, _i, _p, _p, _i, _i]
        R.mia_matvec_scalar.argtypes = [_p, _p, _i, _p, _p, _i, _i]
        R.ref_moe_layer.argtypes = [_i, _i, _i, _i, _i, _f, _i, _p, _p, _p, _p,
                                    ctypes.c_size_t, _p, _p, _p, _p, _p]
        _REF = R
    return _REF


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---- thin numpy wrappers ---------------------------------------------------

def quantize_row_q8(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // QK * BLOCK_BYTES, dtype=np.uint8)
    lib().orc_quantize_row_q8(_ptr(x), _ptr(out), x.size)
    return out


def dequantize_row_q8(blocks, n):
    out = np.zeros(n, dtype=np.float32)
    lib().orc_dequantize_row(1, _ptr(blocks), _ptr(out), n)
    return out


def matvec(w, wtype, x, rows, cols):
    """out = W x with the reference's scalar semantics (wtype 0 F32, 1 Q8_0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(rows, dtype=np.float32)
    xq = np.zeros(max(cols // QK, 1) * BLOCK_BYTES, dtype=np.uint8)
    lib().orc_matvec(_ptr(out), _ptr(w), wtype, _ptr(x), _ptr(xq), rows, cols)
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_rmsnorm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
    return out


def softmax(x):
    x = np.array(x, dtype=np.float32)
    lib().orc_softmax(_ptr(x), x.size)
    return x


def top_k(p, k):
    p = np.ascontiguousarray(p, dtype=np.float32)
    idx = np.zeros(k, dtype=np.int32)
    lib().orc_top_k(_ptr(p), p.size, k, _ptr(idx))
    return idx


def blob_bytes(d):
    return lib().orc_blob_bytes(ctypes.byref(d))


def off_up(d):
    return lib().orc_off_up(ctypes.byref(d))


def off_down(d):
    return lib().orc_off_down(ctypes.byref(d))


def synth_x(seed, T, dim):
    x = np.zeros((T, dim), dtype=np.float32)
    lib().orc_synth_x(seed, T, dim, _ptr(x))
    return x


def synth_router(seed, layer, d):
    w = np.zeros((d.n_experts, d.dim), dtype=np.float32)
    lib().orc_synth_router(seed, layer, ctypes.byref(d), _ptr(w))
    return w


def synth_expert_blob(seed, layer, expert, d):
    b = np.zeros(blob_bytes(d), dtype=np.uint8)
    lib().orc_synth_expert_blob(seed, layer, expert, ctypes.byref(d), _ptr(b))
    return b


def _blob_ptrs(blobs, n):
    arr = (ctypes.c_void_p * n)()
    for i, b in enumerate(blobs):
        arr[i] = None if b is None else b.ctypes.data
    return arr


def route(logits, k, norm_topk=1):
    """Softmax + top-k + gate weights (forward.c:176-181). Returns (idx, w, p)."""
    p = np.array(logits, dtype=np.float32)
    idx = np.zeros(k, dtype=np.int32)
    w = np.zeros(k, dtype=np.float32)
    lib().orc_route(_ptr(p), p.size, k, norm_topk, _ptr(idx), _ptr(w))
    return idx, w, p


def moe_layer(d, x, ffn_norm, router, blobs, bias=None, nthreads=1):
    """One layer on x[T][dim] (copied). blobs: list of E arrays (or None).
    Returns (x_out, idx, w, logits, xn)."""
    x = np.array(x, dtype=np.float32, order="C", ndmin=2)
    T = x.shape[0]
    idx = np.zeros((T, d.n_active), dtype=np.int32)
    w = np.zeros((T, d.n_active), dtype=np.float32)
    logits = np.zeros((T, d.n_experts), dtype=np.float32)
    xn = np.zeros((T, d.dim), dtype=np.float32)
    ptrs = _blob_ptrs(blobs, d.n_experts)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_moe_layer(ctypes.byref(d), T, _ptr(x), _ptr(ffn_norm), _ptr(router),
                             _ptr(bias), ptrs, _ptr(idx), _ptr(w), _ptr(logits), _ptr(xn),
                             nthreads)
    if rc != 0:
        raise RuntimeError("orc_moe_layer failed (%d)" % rc)
    return x, idx, w, logits, xn


def moe_layer_bucketed(d, x, ffn_norm, router, blobs, bias=None, nthreads=1):
    """The same layer as moe_layer (same bits) computed expert by expert, for
    large T. Returns (x_out, idx, w, logits)."""
    x = np.array(x, dtype=np.float32, order="C", ndmin=2)
    T = x.shape[0]
    idx = np.zeros((T, d.n_active), dtype=np.int32)
    w = np.zeros((T, d.n_active), dtype=np.float32)
    logits = np.zeros((T, d.n_experts), dtype=np.float32)
    ptrs = _blob_ptrs(blobs, d.n_experts)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_moe_layer_bucketed(ctypes.byref(d), T, _ptr(x),
                                      _ptr(np.ascontiguousarray(ffn_norm, dtype=np.float32)),
                                      _ptr(np.ascontiguousarray(router, dtype=np.float32)),
                                      _ptr(bias), ptrs, _ptr(idx), _ptr(w), _ptr(logits),
                                      nthreads)
    if rc != 0:
        raise RuntimeError("orc_moe_layer_bucketed failed (%d)" % rc)
    return x, idx, w, logits


def route_tokens(d, x, ffn_norm, router, bias=None, nthreads=1):
    """Routing only (rmsnorm, router chains, softmax, top-K, gate weights) of
    every token of x[T][dim]: the layer without its experts. Returns
    (idx, w, logits)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    idx = np.zeros((T, d.n_active), dtype=np.int32)
    w = np.zeros((T, d.n_active), dtype=np.float32)
    logits = np.zeros((T, d.n_experts), dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_route_tokens(ctypes.byref(d), T, _ptr(x),
                                _ptr(np.ascontiguousarray(ffn_norm, dtype=np.float32)),
                                _ptr(np.ascontiguousarray(router, dtype=np.float32)),
                                _ptr(bias), _ptr(idx), _ptr(w), _ptr(logits), nthreads)
    if rc != 0:
        raise RuntimeError("orc_route_tokens failed (%d)" % rc)
    return idx, w, logits


def model_step(model, kc, vc, max_seq, token, pos, nthreads=1):
    """orc_model_step: logits[vocab] of the token at pos (kc/vc: the KV
    cache, [L][max_seq][kv_dim] float32, updated in place), and the residual
    after the last layer."""
    logits = np.zeros(model.vocab, np.float32)
    x = np.zeros(model.moe.dim, np.float32)
    rc = lib().orc_model_step(ctypes.byref(model), _ptr(kc), _ptr(vc), max_seq, token, pos,
                              _ptr(logits), _ptr(x), nthreads)
    if rc != 0:
        raise RuntimeError("orc_model_step failed (%d)" % rc)
    return logits, x


def rope_row(x, pos, theta):
    x = np.array(x, dtype=np.float32)
    lib().orc_rope_row(_ptr(x), x.size, pos, theta)
    return x


def ref_model_logits(path, tokens, max_seq, n_slots):
    """The reference's own mia_model_step over a .mia file (oracle/_ref):
    logits[len(tokens)][vocab]."""
    import struct
    with open(path, "rb") as f:
        vocab = struct.unpack("<I", f.read(36)[32:36])[0]
    toks = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.zeros((toks.size, vocab), np.float32)
    err = ctypes.create_string_buffer(256)
    R = ref()
    R.ref_model_logits.argtypes = [ctypes.c_char_p, _i, _i, _i, _p, _p, ctypes.c_char_p,
                                   ctypes.c_size_t]
    rc = R.ref_model_logits(path.encode(), max_seq, n_slots, toks.size, _ptr(toks), _ptr(out),
                            err, 256)
    if rc != 0:
        raise RuntimeError("ref_model_logits failed (%d): %s" % (rc, err.value.decode()))
    return out


def moe_stack(d, x, ffn_norm, router, blobs, nthreads=1):
    """ffn_norm[L][dim], router[L][E][dim], blobs: list of L*E arrays."""
    x = np.array(x, dtype=np.float32, order="C", ndmin=2)
    L = ffn_norm.shape[0]
    ptrs = _blob_ptrs(blobs, L * d.n_experts)
    rc = lib().orc_moe_stack(ctypes.byref(d), L, x.shape[0], _ptr(x),
                             _ptr(np.ascontiguousarray(ffn_norm, dtype=np.float32)),
                             _ptr(np.ascontiguousarray(router, dtype=np.float32)), ptrs,
                             nthreads)
    if rc != 0:
        raise RuntimeError("orc_moe_stack failed (%d)" % rc)
    return x


def dispatch(idx, E):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    counts = np.zeros(E, dtype=np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    perm = np.zeros(T * K, dtype=np.int32)
    pos = np.zeros(T * K, dtype=np.int32)
    rc = lib().orc_dispatch(_ptr(idx), T, K, E, _ptr(counts), _ptr(offsets), _ptr(perm),
                            _ptr(pos))
    if rc != 0:
        raise RuntimeError("orc_dispatch failed")
    return counts, offsets, perm, pos


def ref_moe_layer(d, x, ffn_norm, router, blobs):
    """The reference's own moe() (oracle/_ref). Returns
    (x_out, idx_loaded, idx, w, logits, xn)."""
    x = np.array(x, dtype=np.float32, order="C", ndmin=2)
    T = x.shape[0]
    K, E = d.n_active, d.n_experts
    idx_loaded = np.zeros((T, K), dtype=np.int32)
    idx = np.zeros((T, K), dtype=np.int32)
    w = np.zeros((T, K), dtype=np.float32)
    logits = np.zeros((T, E), dtype=np.float32)
    xn = np.zeros((T, d.dim), dtype=np.float32)
    ptrs = _blob_ptrs(blobs, E)
    rc = ref().ref_moe_layer(d.dim, E, K, d.expert_hidden, d.norm_topk, d.norm_eps, T,
                             _ptr(x), _ptr(ffn_norm), _ptr(router), ptrs, blob_bytes(d),
                             _ptr(idx_loaded), _ptr(idx), _ptr(w), _ptr(logits), _ptr(xn))
    if rc != 0:
        raise RuntimeError("ref_moe_layer failed (%d)" % rc)
    return x, idx_loaded, idx, w, logits, xn


def sample(logits, temperature, top_p, seed, draws):
    """orc_sample: `draws` tokens from one sampler state over the same
    logits (float32[n])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    s = Sampler()
    lib().orc_sampler_init(ctypes.byref(s), temperature, top_p, lg.size, seed)
    return [lib().orc_sample(ctypes.byref(s), _ptr(lg)) for _ in range(draws)]


def ref_sample(logits, temperature, top_p, seed, draws):
    """The reference's own mia_sample (oracle/_ref), as `sample`."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.zeros(draws, np.int32)
    R = ref()
    R.ref_sample.argtypes = [_p, _i, _f, _f, _u64, _i, _p]
    if R.ref_sample(_ptr(lg), lg.size, temperature, top_p, seed, draws, _ptr(out)) != 0:
        raise RuntimeError("ref_sample failed")
    return out.tolist()
