""".mia model files into the HBM table (mia_file_probe, mia_moe_load_file).

CPU: the header and dense-section checks of mia_file_probe on files the
test writer lays out as the reference converter does (tests/mia_writer.py),
and every rejection the reference reader makes (src/storage/mia_file.c:
49-61,88-106) plus truncation. GPU: the file-filled table is bit-identical
to the file's blobs and to a table filled through the loader port from the
same file (the reference's streamed == resident rule,
tools/e2e/e2e_test.go:114-122), and layers computed from it are bit-equal to
the oracle's on the file's norms and routers.
"""
import ctypes
import struct
import sys

import numpy as np
import pytest

import motoria_amd as M
import mia_writer as MW


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make_file(oracle, path, cfg, wtype=MW.Q8_0, seed=7):
    return MW.synthetic(oracle, path, cfg, wtype, seed)


@pytest.fixture(scope="module")
def tiny_file(oracle, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("mia") / "tiny.mia")
    return path, make_file(oracle, path, MW.TINY)


# ---- probe (CPU) ----------------------------------------------------------------

def test_probe_reads_the_header_and_walks_the_dense_section(tiny_file):
    path, lay = tiny_file
    info, err = M.file_probe(path)
    assert info is not None, err
    cfg = MW.TINY
    for k in ("dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "n_experts",
              "n_active", "expert_hidden", "norm_topk"):
        assert getattr(info, k) == cfg[k], k
    assert info.version == 1 and info.wtype == MW.Q8_0
    assert info.dense_offset == MW.HEADER_REGION and info.dense_size == lay["dense_size"]
    assert info.experts_offset == lay["experts_offset"]
    assert info.expert_blob_size == lay["blob"]
    assert (info.off_up, info.off_down) == (lay["off_up"], lay["off_down"])
    assert (info.tok_offset, info.tok_size) == (lay["tok_offset"], 3)
    for l in range(cfg["n_layers"]):
        fn, rt = M.file_layer_offsets(info, l)
        assert fn == MW.HEADER_REGION + lay["entries"]["blk.%d.ffn_norm" % l][4]
        assert rt == MW.HEADER_REGION + lay["entries"]["blk.%d.router" % l][4]
    with pytest.raises(ValueError):
        M.file_layer_offsets(info, cfg["n_layers"])


def test_probe_f32_file_geometry(oracle, tmp_path):
    path = str(tmp_path / "f32.mia")
    lay = make_file(oracle, path, MW.TINY, wtype=MW.F32)
    info, err = M.file_probe(path)
    assert info is not None, err
    assert info.wtype == MW.F32 and info.dense_size == lay["dense_size"]
    eh, d = MW.TINY["expert_hidden"], MW.TINY["dim"]
    assert info.off_up == MW.align(eh * d * 4, 64) and info.off_down == 2 * info.off_up


def _patched(src, dst, offset, fmt, value):
    data = bytearray(open(src, "rb").read())
    struct.pack_into(fmt, data, offset, value)
    open(dst, "wb").write(bytes(data))


# (header byte offset, struct format, value, expected message)
BAD_HEADERS = [
    (0, "<4s", b"MIA2", "not a MIA v1 file"),
    (4, "<I", 2, "not a MIA v1 file"),
    (8, "<I", 2, "unsupported model shape"),          # weight type
    (24, "<I", 0, "unsupported model shape"),         # n_kv_heads = 0
    (24, "<I", 3, "unsupported model shape"),         # n_heads % n_kv_heads
    (40, "<I", 9, "unsupported model shape"),         # n_active > n_experts
    (28, "<I", 15, "unsupported model shape"),        # odd head_dim
    (12, "<I", 48, "unsupported model shape"),        # dim % 32
    (44, "<I", 40, "unsupported model shape"),        # expert_hidden % 32
    (72, "<Q", 0, "dense layout mismatch"),           # dense_size
    (88, "<Q", 4096, "expert blob too small"),        # expert_blob_size
    (80, "<Q", 1 << 40, "truncated"),                 # experts beyond the end
]


@pytest.mark.parametrize("offset,fmt,value,msg", BAD_HEADERS)
def test_probe_rejects(tiny_file, tmp_path, offset, fmt, value, msg):
    path, _ = tiny_file
    bad = str(tmp_path / "bad.mia")
    _patched(path, bad, offset, fmt, value)
    info, err = M.file_probe(bad)
    assert info is None and msg in err, err


def test_probe_rejects_truncated_and_missing_files(tiny_file, tmp_path):
    path, lay = tiny_file
    data = open(path, "rb").read()
    cut = str(tmp_path / "cut.mia")
    open(cut, "wb").write(data[:lay["experts_offset"] + lay["blob"]])
    info, err = M.file_probe(cut)
    assert info is None and "truncated" in err
    open(cut, "wb").write(data[:100])
    assert M.file_probe(cut)[0] is None
    info, err = M.file_probe(str(tmp_path / "absent.mia"))
    assert info is None and "open" in err


# ---- load into the HBM table (GPU) --------------------------------------------------

def _handle(cfg, max_tokens):
    shape = dict(dim=cfg["dim"], n_experts=cfg["n_experts"], n_active=cfg["n_active"],
                 expert_hidden=cfg["expert_hidden"], norm_topk=cfg["norm_topk"],
                 norm_eps=cfg["norm_eps"])
    return M.Moe(n_layers=cfg["n_layers"], max_tokens=max_tokens, device=0, **shape)


def _file_tensors(path, lay, cfg):
    norms = [MW.read_dense(path, lay, "blk.%d.ffn_norm" % l)[0] for l in range(cfg["n_layers"])]
    routers = [MW.read_dense(path, lay, "blk.%d.router" % l) for l in range(cfg["n_layers"])]
    return norms, routers


def _check_file_handle(oracle, path, lay, cfg, T, seed):
    d = oracle.dims(dim=cfg["dim"], n_experts=cfg["n_experts"], n_active=cfg["n_active"],
                    expert_hidden=cfg["expert_hidden"], norm_topk=cfg["norm_topk"],
                    norm_eps=cfg["norm_eps"])
    norms, routers = _file_tensors(path, lay, cfg)
    a = _handle(cfg, T)
    b = _handle(cfg, T)
    try:
        a.load_file(path)
        # the same file through the loader port (the reference's streamed path)
        with open(path, "rb") as f:
            def load(l, e, dst):
                f.seek(lay["experts_offset"] + (l * cfg["n_experts"] + e) * lay["blob"])
                blob = f.read(lay["blob"])
                ctypes.memmove(dst, blob, len(blob))
                return 0
            b.load_experts(load)
        for l in range(cfg["n_layers"]):
            b.set_layer(l, norms[l], routers[l])
        for l in range(cfg["n_layers"]):
            for e in range(cfg["n_experts"]):
                want = MW.read_blob(path, lay, cfg, l, e)
                assert np.array_equal(a.read_expert(l, e), want), "expert (%d, %d)" % (l, e)
        x = oracle.synth_x(seed, T, d.dim)
        for l in range(cfg["n_layers"]):
            xa, ia, wa, la = a.layer(l, x)
            xb, ib, wb, lb = b.layer(l, x)
            blobs = [MW.read_blob(path, lay, cfg, l, e) for e in range(cfg["n_experts"])]
            xo, io, wo, lo, _ = oracle.moe_layer(d, x, norms[l], routers[l], blobs)
            for u, v, w_ in ((xa, xb, xo), (la, lb, lo), (wa, wb, wo)):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
                assert np.array_equal(u.view(np.uint32), w_.view(np.uint32))
            assert np.array_equal(ia, io) and np.array_equal(ib, io)
            say("  layer %d: file-filled == loader-port-filled == oracle (T=%d)" % (l, T))
            x = xo
        return a, b
    except Exception:
        a.close()
        b.close()
        raise


@pytest.mark.gpu
def test_load_file_tiny_matches_loader_port_and_oracle(oracle, tiny_file):
    say("test_load_file_tiny_matches_loader_port_and_oracle")
    path, lay = tiny_file
    a, b = _check_file_handle(oracle, path, lay, MW.TINY, 48, 61)
    a.close()
    b.close()


@pytest.mark.gpu
def test_load_file_qwen_layer(oracle, tmp_path):
    """One layer of the Qwen3-30B-A3B MoE shape (attention tensors of its
    shape, a small vocabulary): the file-filled table, the one-token decode
    launch and a 16-token layer bit-equal to the oracle."""
    say("test_load_file_qwen_layer")
    cfg = dict(dim=2048, n_layers=1, n_heads=32, n_kv_heads=4, head_dim=128, vocab=64,
               n_experts=128, n_active=8, expert_hidden=768, norm_topk=1, rope_theta=1e6,
               norm_eps=1e-6)
    path = str(tmp_path / "qwen1.mia")
    lay = make_file(oracle, path, cfg, seed=11)
    a, b = _check_file_handle(oracle, path, lay, cfg, 16, 62)
    try:
        d = oracle.dims(**oracle.QWEN3_30B_A3B)
        norms, routers = _file_tensors(path, lay, cfg)
        x0 = oracle.synth_x(63, 1, d.dim)
        x = x0.copy()
        K = d.n_active
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        assert M.lib().mia_moe_layer_ex(a.h, 0, x.ctypes.data, 1, None, idx.ctypes.data,
                                        w.ctypes.data, None) == 0
        assert a.decode_status()[0] == 0
        blobs = [MW.read_blob(path, lay, cfg, 0, e) for e in range(d.n_experts)]
        xo, io, wo, _, _ = oracle.moe_layer(d, x0, norms[0], routers[0], blobs)
        assert np.array_equal(idx, io[0])
        assert np.array_equal(x.view(np.uint32), xo.view(np.uint32))
    finally:
        a.close()
        b.close()


@pytest.mark.gpu
def test_load_file_rejects_f32_and_other_shapes(oracle, tiny_file, tmp_path):
    say("test_load_file_rejects_f32_and_other_shapes")
    path, _ = tiny_file
    f32 = str(tmp_path / "f32.mia")
    make_file(oracle, f32, MW.TINY, wtype=MW.F32)
    h = _handle(MW.TINY, 4)
    try:
        with pytest.raises(RuntimeError, match="Q8_0 experts"):
            h.load_file(f32)
        with pytest.raises(RuntimeError, match="not a MIA v1 file|open"):
            h.load_file(str(tmp_path / "absent.mia"))
    finally:
        h.close()
    other = _handle(dict(MW.TINY, n_experts=16), 4)
    try:
        with pytest.raises(RuntimeError, match="differs from the handle"):
            other.load_file(path)
    finally:
        other.close()
