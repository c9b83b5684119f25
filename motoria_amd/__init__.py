"""motoria_amd: MI355X-native Qwen3-30B-A3B Q8_0 MoE FFN path.

The product is the C-ABI library motoria_amd/libmotoria.so (gfx950 HIP
kernels + the C99 host library keeping motorIa's engine API). This module
binds it with ctypes for tests and benchmarks. There is no Python or CPU
implementation of the path: importing works without a GPU, but every call
that computes goes to the library and fails loudly when it or the GPU is
missing.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmotoria.so")
_LIB = None

_i = ctypes.c_int
_f = ctypes.c_float
_p = ctypes.c_void_p
_sz = ctypes.c_size_t
_u64 = ctypes.c_uint64

MHIP_FORCE_SEQ_RMS = 1
MHIP_FORCE_EXACT_ROUTER = 2
MHIP_DECODE_TRACE = 4
MHIP_EXACT_EXPERTS = 8
MHIP_DECODE_FORCE_ABORT = 16
MHIP_DECODE_CHAINS_FIRST = 32
MHIP_ATTN_FORCE_ABORT = 64
MHIP_CHAIN_SUM, MHIP_CHAIN_GE, MHIP_CHAIN_GT = 0, 1, 2
MHIP_MODEL_PER_LAYER = 128
MHIP_DECODE_CERTIFIED = 256
MHIP_FAST_DOWN = 512
MHIP_MODEL_STACK_MAX_SEQ = 8192  # longest context of the model stack (mia_hip.h)
DECODE_MAX_LAYERS = 256  # MHIP_DECODE_MAX_LAYERS
GEMM_MIN_A = 2048  # MHIP_GEMM_MIN_A
TRACE_L0, TRACE_NL, TRACE_SLOTS = 8, 8, 48  # decode trace window (MHIP_TRACE_* in mia_hip.h)
STAGES = ["rmsnorm", "router", "dispatch", "gateup", "down", "combine", "decode"]


class MoeConfig(ctypes.Structure):
    _fields_ = [("dim", _i), ("n_layers", _i), ("n_experts", _i), ("n_active", _i),
                ("expert_hidden", _i), ("norm_topk", _i), ("norm_eps", _f),
                ("max_tokens", _i), ("device", _i)]


class Dims(ctypes.Structure):
    _fields_ = [("dim", _i), ("n_experts", _i), ("n_active", _i), ("expert_hidden", _i),
                ("norm_topk", _i), ("norm_eps", _f)]


class Layout(ctypes.Structure):
    _fields_ = [("gate_q", _sz), ("up_q", _sz), ("down_q", _sz), ("gate_s", _sz),
                ("up_s", _sz), ("down_s", _sz), ("gate_st", _sz), ("up_st", _sz),
                ("down_st", _sz), ("expert_bytes", _sz)]


class Scratch(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("xn", "xq", "xs", "logits", "idx", "w", "counts", "offsets",
                                  "perm", "pos", "groups", "h", "tmp", "status", "xdq",
                                  "hdq", "gtile", "xsb", "hq", "hs", "glight")]


class AttnDims(ctypes.Structure):
    _fields_ = [("dim", _i), ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i),
                ("norm_eps", _f)]


class Sampler(ctypes.Structure):
    """mhip_sampler (include/mia_hip.h)."""
    _fields_ = [("temperature", _f), ("top_p", _f), ("n", _i), ("rng", _u64)]


class FileInfo(ctypes.Structure):
    """mia_file_info (include/mia/moe.h): a .mia header and blob offsets."""
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "version", "wtype", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab",
        "n_experts", "n_active", "expert_hidden", "norm_topk")] + [
        ("rope_theta", _f), ("norm_eps", _f)] + [(n, ctypes.c_uint64) for n in (
            "dense_offset", "dense_size", "experts_offset", "expert_blob_size", "tok_offset",
            "tok_size", "off_up", "off_down")]


def file_probe(path):
    """mia_file_probe: (FileInfo, None) or (None, error message)."""
    info = FileInfo()
    err = ctypes.create_string_buffer(512)
    if lib().mia_file_probe(path.encode(), ctypes.byref(info), err, 512) != 0:
        return None, err.value.decode()
    return info, None


def file_layer_offsets(info, layer):
    fn, rt = ctypes.c_uint64(), ctypes.c_uint64()
    if lib().mia_file_layer_offsets(ctypes.byref(info), layer, ctypes.byref(fn),
                                    ctypes.byref(rt)) != 0:
        raise ValueError("layer %d out of range" % layer)
    return fn.value, rt.value


# Every function the library exports, with its ctypes signature. tests check
# this list against the declarations in include/.
SIGNATURES = {
    # include/mia_hip.h
    "mhip_layout_of": (_i, [ctypes.POINTER(Dims), ctypes.POINTER(Layout)]),
    "mhip_device_count": (_i, []),
    "mhip_open": (_i, [ctypes.POINTER(_p), _i, ctypes.c_char_p, _sz]),
    "mhip_close": (None, [_p]),
    "mhip_error": (ctypes.c_char_p, [_p]),
    "mhip_malloc": (_p, [_p, _sz]),
    "mhip_free": (_i, [_p, _p]),
    "mhip_h2d": (_i, [_p, _p, _p, _sz]),
    "mhip_d2h": (_i, [_p, _p, _p, _sz]),
    "mhip_d2d": (_i, [_p, _p, _p, _sz]),
    "mhip_host_malloc": (_p, [_p, _sz]),
    "mhip_host_free": (_i, [_p, _p]),
    "mhip_h2d_async": (_i, [_p, _p, _p, _sz]),
    "mhip_d2h_async": (_i, [_p, _p, _p, _sz]),
    "mhip_zero": (_i, [_p, _p, _sz]),
    "mhip_sync": (_i, [_p]),
    "mhip_mark": (_i, [_p, _i]),
    "mhip_elapsed": (_i, [_p, _i, _i, ctypes.POINTER(_f)]),
    "mhip_mark_wait": (_i, [_p, _i]),
    "mhip_stage_timing": (_i, [_p, ctypes.c_uint, _i]),
    "mhip_stage_time": (_i, [_p, _i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i)]),
    "mhip_matrix_layers": (ctypes.c_ulonglong, [_p]),
    "mhip_table_repack": (_i, [_p, ctypes.POINTER(Dims), _p, _i, ctypes.POINTER(_i), _i, _p,
                               _sz, _sz, _sz]),
    "mhip_table_unpack": (_i, [_p, ctypes.POINTER(Dims), _p, _i, _i, _p, _sz, _sz, _sz]),
    "mhip_table_synth": (_i, [_p, ctypes.POINTER(Dims), _p, _u64, _i, _i]),
    "mhip_router_synth": (_i, [_p, ctypes.POINTER(Dims), _p, _p, _u64, _i]),
    "mhip_router_transpose": (_i, [_p, ctypes.POINTER(Dims), _p, _p]),
    "mhip_router_decode_layout": (_i, [_p, ctypes.POINTER(Dims), _p, _p]),
    "mhip_synth_f32": (_i, [_p, _p, _sz, _u64, _u64, ctypes.c_double]),
    "mhip_fill_f32": (_i, [_p, _p, _sz, _f]),
    "mhip_scratch_bytes": (_sz, [ctypes.POINTER(Dims), _i]),
    "mhip_scratch_carve": (_i, [ctypes.POINTER(Dims), _i, _p, ctypes.POINTER(Scratch)]),
    "mhip_moe_layer": (_i, [_p, ctypes.POINTER(Dims), ctypes.POINTER(Layout), _p, _p, _p, _p,
                            _p, _i, ctypes.POINTER(Scratch), _i]),
    "mhip_decode_ws_bytes": (_sz, []),
    "mhip_decode_supported": (_i, [_p, ctypes.POINTER(Dims)]),
    "mhip_decode_stack": (_i, [_p, ctypes.POINTER(Dims), ctypes.POINTER(Layout), _p, _p, _p, _p,
                               _p, _p, _i, _p, _p, _p, _i]),
    "mhip_decode_stack_noalloc": (_i, [_p, ctypes.POINTER(Dims), ctypes.POINTER(Layout), _p, _p,
                                       _p, _p, _p, _p, _i, _p, _p, _p, _i]),
    "mhip_decode_status": (_i, [_p, _p, ctypes.POINTER(_i)]),
    "mhip_decode_trace": (_i, [_p, _p, _p]),
    "mhip_attention_scratch_bytes": (_sz, [ctypes.POINTER(AttnDims), _i]),
    "mhip_attention": (_i, [_p, ctypes.POINTER(AttnDims), _p, _p, _p, _p, _p, _p, _p, _p, _p,
                            _p, _i, _i, _p, _p, _p, _i]),
    "mhip_attention_batch_scratch_bytes": (_sz, [ctypes.POINTER(AttnDims), _i, _i]),
    "mhip_attention_batch": (_i, [_p, ctypes.POINTER(AttnDims), _p, _p, _p, _p, _p, _p, _p, _p,
                                  _p, _p, _i, _i, _i, _p, _p, _p, _i]),
    "mhip_attention_pack_bytes": (_sz, [ctypes.POINTER(AttnDims)]),
    "mhip_attention_pack": (_i, [_p, ctypes.POINTER(AttnDims), _p, _p, _p, _p, _p]),
    "mhip_output_head": (_i, [_p, ctypes.POINTER(AttnDims), _p, _p, _i, _p, _p, _p, _i]),
    "mhip_attention_layer_ws_bytes": (_sz, []),
    "mhip_attention_layer_trace": (_i, [_p, _p, _p]),
    "mhip_attention_layer_supported": (_i, [_p, ctypes.POINTER(AttnDims), _i]),
    "mhip_attention_layer": (_i, [_p, ctypes.POINTER(AttnDims), _p, _p, _p, _p, _p, _p, _p, _p,
                                  _p, _p, _i, _i, _p, _p, _p, _p, _p, _i]),
    "mhip_graph_begin": (_i, [_p]),
    "mhip_graph_end": (_i, [_p, ctypes.POINTER(_p)]),
    "mhip_graph_launch": (_i, [_p, _p]),
    "mhip_graph_destroy": (None, [_p]),
    "mhip_sampler_init": (None, [ctypes.POINTER(Sampler), _f, _f, _i, _u64]),
    "mhip_sample_scratch_bytes": (_sz, [_i]),
    "mhip_sample": (_i, [_p, ctypes.POINTER(Sampler), _p, _p, _p]),
    "mhip_chain_f32": (_i, [_p, _p, _i, _i, _f, _p]),
    "mhip_model_stack_ws_bytes": (_sz, []),
    "mhip_model_stack_supported": (_i, [_p, _p, _p, _i]),
    "mhip_model_stack": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _p, _i, _p,
                              _p, _i]),
    "mhip_quantize_q8": (_i, [_p, _p, _p, _i]),
    "mhip_dequantize_q8": (_i, [_p, _p, _p, _i]),
    "mhip_matvec": (_i, [_p, _p, _p, _i, _p, _p, _i, _i]),
    # include/mia/quant.h, include/mia/matmul.h
    "mia_row_bytes": (_sz, [_i, _i]),
    "mia_quantize_row_q8": (None, [_p, _p, _i]),
    "mia_dequantize_row": (None, [_i, _p, _p, _i]),
    "mia_matvec": (None, [_p, _p, _i, _p, _p, _i, _i]),
    "mia_matvec_scalar": (None, [_p, _p, _i, _p, _p, _i, _i]),
    # include/mia/matvec_cache.h
    "mia_matvec_register": (_i, [_p, _i, _i, _i]),
    "mia_matvec_unregister": (_i, [_p]),
    # include/mia/tensor_error.h
    "mia_tensor_error": (ctypes.c_char_p, []),
    # include/mia/moe.h
    "mia_moe_open": (_i, [ctypes.POINTER(_p), ctypes.POINTER(MoeConfig), ctypes.c_char_p, _sz]),
    "mia_moe_close": (None, [_p]),
    "mia_moe_error": (ctypes.c_char_p, [_p]),
    "mia_moe_blob_bytes": (_sz, [_p]),
    "mia_moe_off_up": (_sz, [_p]),
    "mia_moe_off_down": (_sz, [_p]),
    "mia_moe_load_experts": (_i, [_p, _p, _p]),
    "mia_moe_load_expert": (_i, [_p, _i, _i, _p]),
    "mia_moe_read_expert": (_i, [_p, _i, _i, _p]),
    "mia_moe_set_layer": (_i, [_p, _i, _p, _p]),
    "mia_moe_synth": (_i, [_p, _u64]),
    "mia_moe_layer": (_i, [_p, _i, _p, _i]),
    "mia_moe_layer_ex": (_i, [_p, _i, _p, _i, _p, _p, _p, _p]),
    "mia_moe_stack": (_i, [_p, _i, _i, _p, _i]),
    "mia_moe_layer_dev": (_i, [_p, _i, _p, _i, _p]),
    "mia_moe_stack_dev": (_i, [_p, _i, _i, _p, _i]),
    "mia_moe_stack_graph": (_i, [_p, _i, _i, _p, _i]),
    "mia_file_probe": (_i, [ctypes.c_char_p, ctypes.POINTER(FileInfo), ctypes.c_char_p, _sz]),
    "mia_file_layer_offsets": (_i, [ctypes.POINTER(FileInfo), _i,
                                    ctypes.POINTER(ctypes.c_uint64),
                                    ctypes.POINTER(ctypes.c_uint64)]),
    "mia_moe_load_file": (_i, [_p, ctypes.c_char_p]),
    "mia_moe_decode": (_i, [_p, _i, _i, _p, _p, _p, _p]),
    "mia_moe_decode_dev": (_i, [_p, _i, _i, _p, _p]),
    "mia_moe_decode_status": (_i, [_p, ctypes.POINTER(_i)]),
    "mia_moe_decode_trace": (_i, [_p, _p]),
    "mia_moe_gpu": (_p, [_p]),
    "mia_moe_scratch": (ctypes.POINTER(Scratch), [_p]),
    "mia_moe_set_flags": (None, [_p, _i]),
    "mia_moe_status": (_i, [_p, ctypes.POINTER(_i)]),
    # include/mia/model_gpu.h
    "mia_gpu_model_open": (_i, [ctypes.POINTER(_p), ctypes.c_char_p, _i, _i, ctypes.c_char_p,
                                _sz]),
    "mia_gpu_model_synth": (_i, [ctypes.POINTER(_p), ctypes.POINTER(FileInfo), _i, _i, _u64,
                                 ctypes.c_char_p, _sz]),
    "mia_gpu_model_close": (None, [_p]),
    "mia_gpu_model_error": (ctypes.c_char_p, [_p]),
    "mia_gpu_model_vocab": (_i, [_p]),
    "mia_gpu_model_step": (ctypes.POINTER(_f), [_p, _i, _i]),
    "mia_gpu_model_step_sample": (_i, [_p, _i, _i, ctypes.POINTER(Sampler)]),
    "mia_gpu_model_feed": (_i, [_p, _i, _i]),
    "mia_gpu_model_prefill": (_i, [_p, _p, _i, _i]),
    "mia_gpu_model_sample": (_i, [_p, ctypes.POINTER(Sampler)]),
    "mia_gpu_model_info": (ctypes.POINTER(FileInfo), [_p]),
    "mia_gpu_model_set_flags": (None, [_p, _i]),
    "mia_gpu_model_aborts": (_i, [_p]),
    "mia_gpu_model_trace": (_i, [_p, _p]),
    # include/mia/serve.h
    "mia_bpe_open": (_i, [ctypes.POINTER(_p), _p, _sz]),
    "mia_bpe_close": (None, [_p]),
    "mia_bpe_encode": (_i, [_p, ctypes.c_char_p, _p, _i]),
    "mia_bpe_piece": (ctypes.POINTER(ctypes.c_ubyte), [_p, _i, ctypes.POINTER(_i)]),
    "mia_bpe_is_stop": (_i, [_p, _i]),
    "mia_bpe_vocab": (_i, [_p]),
    "mia_bpe_im_start": (_i, [_p]),
    "mia_chat_turn_text": (_p, [ctypes.c_char_p, _i, _i]),
    "mia_serve": (_i, [ctypes.c_char_p, _i, _u64, _i, _p, _p]),
}

# The storage port type (include/mia/expert_cache.h).
LOADER = ctypes.CFUNCTYPE(_i, _p, _i, _i, _p)


def lib():
    """Load libmotoria.so (raises if it is not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("motoria_amd/libmotoria.so is not built; run "
                               "`python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def device_count():
    return lib().mhip_device_count()


def _ptr(a):
    return None if a is None else a.ctypes.data


QWEN3_30B_A3B = dict(dim=2048, n_experts=128, n_active=8, expert_hidden=768, norm_topk=1,
                     norm_eps=1e-6)


class Moe:
    """A mia_moe handle: resident expert table + scratch on one GPU."""

    def __init__(self, n_layers, max_tokens, device=0, **shape):
        shape = dict(QWEN3_30B_A3B, **shape)
        self.shape = shape
        self.n_layers = n_layers
        self.max_tokens = max_tokens
        cfg = MoeConfig(dim=shape["dim"], n_layers=n_layers, n_experts=shape["n_experts"],
                        n_active=shape["n_active"], expert_hidden=shape["expert_hidden"],
                        norm_topk=shape["norm_topk"], norm_eps=shape["norm_eps"],
                        max_tokens=max_tokens, device=device)
        h = _p()
        err = ctypes.create_string_buffer(512)
        if lib().mia_moe_open(ctypes.byref(h), ctypes.byref(cfg), err, 512) != 0:
            raise RuntimeError("mia_moe_open: " + err.value.decode())
        self.h = h
        self.gpu = lib().mia_moe_gpu(h)
        self.dims = Dims(shape["dim"], shape["n_experts"], shape["n_active"],
                         shape["expert_hidden"], shape["norm_topk"], shape["norm_eps"])

    def close(self):
        if self.h:
            lib().mia_moe_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError("%s: %s" % (what, lib().mia_moe_error(self.h).decode()))

    # -- geometry / weights
    @property
    def blob_bytes(self):
        return lib().mia_moe_blob_bytes(self.h)

    @property
    def off_up(self):
        return lib().mia_moe_off_up(self.h)

    @property
    def off_down(self):
        return lib().mia_moe_off_down(self.h)

    def synth(self, seed):
        self._check(lib().mia_moe_synth(self.h, seed), "mia_moe_synth")

    def load_expert(self, layer, expert, blob):
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        self._check(lib().mia_moe_load_expert(self.h, layer, expert, _ptr(blob)),
                    "mia_moe_load_expert")

    def load_experts(self, loader_fn):
        """loader_fn(layer, expert, dst_ptr) -> int, the storage port."""
        cb = LOADER(lambda ctx, l, e, dst: loader_fn(l, e, dst))
        self._check(lib().mia_moe_load_experts(self.h, cb, None), "mia_moe_load_experts")

    def load_file(self, path):
        """Fill the handle from a .mia file (mia_moe_load_file)."""
        self._check(lib().mia_moe_load_file(self.h, path.encode()), "mia_moe_load_file")

    def read_expert(self, layer, expert):
        out = np.zeros(self.blob_bytes, dtype=np.uint8)
        self._check(lib().mia_moe_read_expert(self.h, layer, expert, _ptr(out)),
                    "mia_moe_read_expert")
        return out

    def set_layer(self, layer, ffn_norm, router):
        ffn_norm = np.ascontiguousarray(ffn_norm, dtype=np.float32)
        router = np.ascontiguousarray(router, dtype=np.float32)
        self._check(lib().mia_moe_set_layer(self.h, layer, _ptr(ffn_norm), _ptr(router)),
                    "mia_moe_set_layer")

    def set_flags(self, flags):
        lib().mia_moe_set_flags(self.h, flags)

    def status(self):
        st = (_i * 4)()
        self._check(lib().mia_moe_status(self.h, st), "mia_moe_status")
        return list(st)

    # -- compute (host pointers)
    def layer(self, layer, x, bias=None):
        """Returns (x_out, idx, w, logits) for x[T][dim]."""
        x = np.array(x, dtype=np.float32, order="C", ndmin=2)
        T = x.shape[0]
        K, E = self.shape["n_active"], self.shape["n_experts"]
        idx = np.zeros((T, K), dtype=np.int32)
        w = np.zeros((T, K), dtype=np.float32)
        logits = np.zeros((T, E), dtype=np.float32)
        bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._check(lib().mia_moe_layer_ex(self.h, layer, _ptr(x), T, _ptr(bias), _ptr(idx),
                                           _ptr(w), _ptr(logits)), "mia_moe_layer_ex")
        return x, idx, w, logits

    def stack(self, l0, l1, x):
        x = np.array(x, dtype=np.float32, order="C", ndmin=2)
        self._check(lib().mia_moe_stack(self.h, l0, l1, _ptr(x), x.shape[0]), "mia_moe_stack")
        return x

    # -- compute (device pointers)
    def layer_dev(self, layer, d_x, T, d_bias=None):
        self._check(lib().mia_moe_layer_dev(self.h, layer, d_x, T, d_bias), "mia_moe_layer_dev")

    def stack_dev(self, l0, l1, d_x, T):
        self._check(lib().mia_moe_stack_dev(self.h, l0, l1, d_x, T), "mia_moe_stack_dev")

    def stack_graph(self, l0, l1, d_x, T):
        self._check(lib().mia_moe_stack_graph(self.h, l0, l1, d_x, T), "mia_moe_stack_graph")

    def decode(self, l0, l1, x, bias=None):
        """One token through layers [l0, l1) in one persistent launch.
        Returns (x_out, idx[l1-l0][K], w[l1-l0][K])."""
        x = np.array(x, dtype=np.float32).reshape(-1).copy()
        K = self.shape["n_active"]
        idx = np.zeros((l1 - l0, K), dtype=np.int32)
        w = np.zeros((l1 - l0, K), dtype=np.float32)
        bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._check(lib().mia_moe_decode(self.h, l0, l1, _ptr(x), _ptr(bias), _ptr(idx), _ptr(w)),
                    "mia_moe_decode")
        return x, idx, w

    def decode_trace(self):
        out = np.zeros((TRACE_NL, 256, TRACE_SLOTS), dtype=np.uint64)
        self._check(lib().mia_moe_decode_trace(self.h, out.ctypes.data), "mia_moe_decode_trace")
        return out

    def decode_dev(self, l0, l1, d_x, d_bias=None):
        self._check(lib().mia_moe_decode_dev(self.h, l0, l1, d_x, d_bias), "mia_moe_decode_dev")

    def decode_status(self):
        st = (_i * 4)()
        self._check(lib().mia_moe_decode_status(self.h, st), "mia_moe_decode_status")
        return list(st)

    def scratch(self):
        return lib().mia_moe_scratch(self.h).contents

    # -- device memory through the handle's context
    def malloc(self, nbytes):
        p = lib().mhip_malloc(self.gpu, nbytes)
        if not p:
            raise RuntimeError("mhip_malloc: " + lib().mhip_error(self.gpu).decode())
        return p

    def free(self, p):
        lib().mhip_free(self.gpu, p)

    def h2d(self, d_dst, arr):
        arr = np.ascontiguousarray(arr)
        if lib().mhip_h2d(self.gpu, d_dst, _ptr(arr), arr.nbytes) != 0:
            raise RuntimeError("mhip_h2d: " + lib().mhip_error(self.gpu).decode())

    def d2h(self, d_src, shape, dtype):
        out = np.zeros(shape, dtype=dtype)
        if lib().mhip_d2h(self.gpu, _ptr(out), d_src, out.nbytes) != 0:
            raise RuntimeError("mhip_d2h: " + lib().mhip_error(self.gpu).decode())
        return out

    def sync(self):
        if lib().mhip_sync(self.gpu) != 0:
            raise RuntimeError("mhip_sync: " + lib().mhip_error(self.gpu).decode())

    def mark(self, slot):
        if lib().mhip_mark(self.gpu, slot) != 0:
            raise RuntimeError("mhip_mark: " + lib().mhip_error(self.gpu).decode())

    def elapsed_ms(self, s0, s1):
        ms = _f()
        if lib().mhip_elapsed(self.gpu, s0, s1, ctypes.byref(ms)) != 0:
            raise RuntimeError("mhip_elapsed: " + lib().mhip_error(self.gpu).decode())
        return ms.value

    def stage_timing(self, stages, max_launches):
        mask = 0
        for st in stages:
            mask |= 1 << STAGES.index(st)
        if lib().mhip_stage_timing(self.gpu, mask, max_launches) != 0:
            raise RuntimeError("mhip_stage_timing: " + lib().mhip_error(self.gpu).decode())

    def stage_time(self, stage):
        ms = ctypes.c_double()
        n = _i()
        if lib().mhip_stage_time(self.gpu, STAGES.index(stage), ctypes.byref(ms),
                                 ctypes.byref(n)) != 0:
            raise RuntimeError("mhip_stage_time: " + lib().mhip_error(self.gpu).decode())
        return ms.value, n.value

    def synth_f32(self, d_out, n, seed, stream, sigma):
        if lib().mhip_synth_f32(self.gpu, d_out, n, seed, stream, sigma) != 0:
            raise RuntimeError("mhip_synth_f32: " + lib().mhip_error(self.gpu).decode())


class Gpu:
    """A bare mhip context (for the tensor-op kernels on device pointers)."""

    def __init__(self, device=0):
        h = _p()
        err = ctypes.create_string_buffer(512)
        if lib().mhip_open(ctypes.byref(h), device, err, 512) != 0:
            raise RuntimeError("mhip_open: " + err.value.decode())
        self.h = h

    def close(self):
        if self.h:
            lib().mhip_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError("%s: %s" % (what, lib().mhip_error(self.h).decode()))

    def malloc(self, nbytes):
        p = lib().mhip_malloc(self.h, nbytes)
        if not p:
            raise RuntimeError("mhip_malloc: " + lib().mhip_error(self.h).decode())
        return p

    def free(self, p):
        lib().mhip_free(self.h, p)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.malloc(max(arr.nbytes, 1))
        self.check(lib().mhip_h2d(self.h, p, _ptr(arr), arr.nbytes), "h2d")
        return p

    def download(self, p, shape, dtype):
        out = np.zeros(shape, dtype=dtype)
        self.check(lib().mhip_d2h(self.h, _ptr(out), p, out.nbytes), "d2h")
        return out


class GpuModel:
    """mia_gpu_model (include/mia/model_gpu.h): the whole model step of a
    Q8_0 .mia file on one GPU."""

    def __init__(self, path, max_seq, device=0, flags=MHIP_FORCE_EXACT_ROUTER, synth=None):
        """Opens the .mia file at `path`, or (path None) generates the model
        of shape `synth` = (dict of header fields, seed) in HBM."""
        h = _p()
        err = ctypes.create_string_buffer(512)
        if path is None:
            cfg, seed = synth
            info = FileInfo(version=1, wtype=1, **{k: v for k, v in cfg.items()
                                                   if k in dict(FileInfo._fields_)})
            rc = lib().mia_gpu_model_synth(ctypes.byref(h), ctypes.byref(info), max_seq, device,
                                           seed, err, 512)
        else:
            rc = lib().mia_gpu_model_open(ctypes.byref(h), path.encode(), max_seq, device, err,
                                          512)
        if rc != 0:
            raise RuntimeError("mia_gpu_model_open: " + err.value.decode())
        self.h = h
        self.vocab = lib().mia_gpu_model_vocab(h)
        self.set_flags(flags)

    def close(self):
        if self.h:
            lib().mia_gpu_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_flags(self, flags):
        lib().mia_gpu_model_set_flags(self.h, flags)

    def aborts(self):
        """Decode launches of the last step that aborted (rerun per stage)."""
        return lib().mia_gpu_model_aborts(self.h)

    def trace(self):
        """Stage timestamps of the last step's model stack launch (flags with
        MHIP_DECODE_TRACE): [TRACE_NL layers][256 workgroups][TRACE_SLOTS]."""
        out = np.zeros((TRACE_NL, 256, TRACE_SLOTS), dtype=np.uint64)
        if lib().mia_gpu_model_trace(self.h, out.ctypes.data):
            raise RuntimeError("mia_gpu_model_trace: " +
                               lib().mia_gpu_model_error(self.h).decode())
        return out

    def step_sample(self, token, pos, sampler):
        """The next token picked on the device (sampler: a Sampler over the
        vocabulary, its rng advanced in place)."""
        r = lib().mia_gpu_model_step_sample(self.h, token, pos, ctypes.byref(sampler))
        if r < 0:
            raise RuntimeError("mia_gpu_model_step_sample: " +
                               lib().mia_gpu_model_error(self.h).decode())
        return r

    def feed(self, token, pos):
        """A prompt step without the output head."""
        if lib().mia_gpu_model_feed(self.h, token, pos) != 0:
            raise RuntimeError("mia_gpu_model_feed: " +
                               lib().mia_gpu_model_error(self.h).decode())

    def prefill(self, tokens, pos):
        """Prompt steps for tokens at pos, pos + 1, ... in batches (no logits)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        if lib().mia_gpu_model_prefill(self.h, t.ctypes.data, len(t), pos) != 0:
            raise RuntimeError("mia_gpu_model_prefill: " +
                               lib().mia_gpu_model_error(self.h).decode())

    def sample(self, sampler):
        """The sampler on the last step's device logits."""
        r = lib().mia_gpu_model_sample(self.h, ctypes.byref(sampler))
        if r < 0:
            raise RuntimeError("mia_gpu_model_sample: " +
                               lib().mia_gpu_model_error(self.h).decode())
        return r

    def step(self, token, pos):
        """Logits (a copy) of `token` at `pos`."""
        r = lib().mia_gpu_model_step(self.h, token, pos)
        if not r:
            raise RuntimeError("mia_gpu_model_step: " +
                               lib().mia_gpu_model_error(self.h).decode())
        return np.ctypeslib.as_array(r, shape=(self.vocab,)).copy()


def sampler(temperature, top_p, n, seed):
    """mhip_sampler_init."""
    s = Sampler()
    lib().mhip_sampler_init(ctypes.byref(s), temperature, top_p, n, seed)
    return s


def sample_dev(gpu, s, d_logits, d_scratch, d_token):
    """mhip_sample on a Gpu context (queued; read d_token after a sync)."""
    gpu.check(lib().mhip_sample(gpu.h, ctypes.byref(s), d_logits, d_scratch, d_token),
              "mhip_sample")


SERVE_PATH = os.path.join(_HERE, "mia-serve")


class Bpe:
    """mia_bpe (include/mia/serve.h): the MTK1 tokenizer of a .mia file."""

    def __init__(self, blob):
        self._blob = bytes(blob)
        h = _p()
        if lib().mia_bpe_open(ctypes.byref(h), self._blob, len(self._blob)) != 0:
            raise ValueError("not a valid MTK1 blob")
        self.h = h

    def close(self):
        if self.h:
            lib().mia_bpe_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text, max_ids=1 << 16):
        """Ids of `text` (str or UTF-8 bytes), or None when more than max_ids
        would be needed."""
        raw = text.encode() if isinstance(text, str) else text
        out = np.zeros(max(max_ids, 1), np.int32)
        n = lib().mia_bpe_encode(self.h, raw, out.ctypes.data, max_ids)
        return None if n < 0 else out[:n].tolist()

    def piece(self, i):
        n = _i()
        p = lib().mia_bpe_piece(self.h, i, ctypes.byref(n))
        return ctypes.string_at(p, n.value)

    def is_stop(self, i):
        return bool(lib().mia_bpe_is_stop(self.h, i))

    def vocab(self):
        return lib().mia_bpe_vocab(self.h)

    def im_start(self):
        return lib().mia_bpe_im_start(self.h)


def chat_turn_text(user, think, continuing):
    """mia_chat_turn_text (freed here)."""
    p = lib().mia_chat_turn_text(user.encode(), think, continuing)
    if not p:
        raise MemoryError("mia_chat_turn_text")
    try:
        return ctypes.string_at(p).decode()
    finally:
        ctypes.CDLL(None).free(ctypes.c_void_p(p))
