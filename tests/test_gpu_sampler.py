"""The token sampler on device logits (mhip_sample, sampler.hip) against the
reference's own picks (tests/golden/sampler.npz, from oracle/_ref) and the
oracle: greedy with NaN, temperature / top-p draws over 2 to 151936 logits,
ties, sanitized top_p, the default seed, the state's advance, and
generation through mia_gpu_model_step_sample."""
import ctypes
import sys

import numpy as np
import pytest

import motoria_amd as M
import mia_writer as MW
from test_golden import sampler_cases

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class DevSampler:
    """Device logits, scratch and token for n logits on one context."""

    def __init__(self, gpu, n):
        self.gpu, self.n = gpu, n
        nb = M.lib().mhip_sample_scratch_bytes(n)
        assert nb > 0
        self.d_scratch = gpu.malloc(nb)
        self.d_logits = gpu.malloc(4 * n)
        self.d_token = gpu.malloc(4)

    def draws(self, logits, t, p, seed, draws):
        lg = np.ascontiguousarray(logits, np.float32)
        assert lg.size == self.n
        self.gpu.check(M.lib().mhip_h2d(self.gpu.h, self.d_logits, lg.ctypes.data, lg.nbytes),
                       "h2d")
        s = M.sampler(t, p, self.n, seed)
        out = []
        for _ in range(draws):
            M.sample_dev(self.gpu, s, self.d_logits, self.d_scratch, self.d_token)
            out.append(int(self.gpu.download(self.d_token, (1,), np.int32)[0]))
        back = self.gpu.download(self.d_logits, lg.shape, np.float32)
        assert np.array_equal(back.view(np.uint32), lg.view(np.uint32)), "logits modified"
        return out, s

    def close(self):
        for p in (self.d_scratch, self.d_logits, self.d_token):
            self.gpu.free(p)


@pytest.fixture(scope="module")
def gpu():
    g = M.Gpu(0)
    yield g
    g.close()


def test_sampler_golden(oracle, gpu):
    say("test_sampler_golden")
    byn = {}
    for name, lg, t, p, seed, draws, want in sampler_cases(oracle):
        n = lg.size
        if n not in byn:
            byn[n] = DevSampler(gpu, n)
        got, _ = byn[n].draws(lg, t, p, seed, draws)
        assert got == want, name
        say("  %-16s n=%-6d T=%-4g top_p=%-6g %4d draws equal" % (name, n, t, p, draws))
    for d in byn.values():
        d.close()


def test_sampler_greedy_nan_and_ties(oracle, gpu):
    say("test_sampler_greedy_nan_and_ties")
    rng = np.random.default_rng(9)
    for n in (1, 2, 3, 255, 256, 257, 70000, 151936):
        ds = DevSampler(gpu, n)
        try:
            for trial in range(6):
                lg = np.round(rng.standard_normal(n) * 2).astype(np.float32)
                if trial >= 2 and n > 3:
                    lg[rng.integers(0, n, max(1, n // 50))] = np.nan
                if trial == 4:
                    lg[0] = np.nan
                if trial == 5 and n > 3:
                    lg[1:] = np.nan
                got, _ = ds.draws(lg, 0.0, 1.0, 1, 1)
                assert got == oracle.sample(lg, 0.0, 1.0, 1, 1), (n, trial)
        finally:
            ds.close()


def test_sampler_no_candidate_and_state(oracle, gpu):
    """NaN logits under temperature (no candidate survives, where the
    reference reads outside its buffer) give the greedy token; every draw
    with temperature > 0 advances the state once, as the reference's."""
    say("test_sampler_no_candidate_and_state")
    n = 1000
    ds = DevSampler(gpu, n)
    try:
        lg = np.random.default_rng(2).standard_normal(n).astype(np.float32)
        lg[17] = np.nan
        got, s = ds.draws(lg, 0.8, 0.9, 77, 5)
        assert got == oracle.sample(lg, 0.8, 0.9, 77, 5)
        o = oracle.Sampler()
        oracle.lib().orc_sampler_init(ctypes.byref(o), 0.8, 0.9, n, 77)
        for _ in range(5):
            oracle.lib().orc_sample(ctypes.byref(o), lg.ctypes.data)
        assert s.rng == o.rng
        # all probabilities equal and below the cutoff of a tiny top_p
        flat = np.zeros(n, np.float32)
        got, _ = ds.draws(flat, 1.0, 1e-6, 5, 3)
        assert got == oracle.sample(flat, 1.0, 1e-6, 5, 3)
    finally:
        ds.close()
    with pytest.raises(RuntimeError, match="outside"):
        s = M.sampler(1.0, 1.0, 0, 1)
        M.sample_dev(gpu, s, ds.d_logits, ds.d_scratch, ds.d_token)
    assert M.lib().mhip_sample_scratch_bytes(0) == 0
    assert M.lib().mhip_sample_scratch_bytes((1 << 21) + 1) == 0


@pytest.mark.parametrize("t,p", [(0.0, 1.0), (0.8, 0.9), (1.3, 1.0)])
def test_model_generation_step_sample(oracle, tmp_path, t, p):
    """Autoregressive generation on the tiny model: each token picked on the
    device by step_sample equals the oracle's pick over the logits of a
    second handle fed the same tokens, and the sampler states agree."""
    say("test_model_generation_step_sample T=%g top_p=%g" % (t, p))
    path = str(tmp_path / "tiny.mia")
    MW.synthetic(oracle, path, MW.TINY, MW.Q8_0, 21)
    n, V = 48, MW.TINY["vocab"]
    a = M.GpuModel(path, n)
    b = M.GpuModel(path, n)
    try:
        s = M.sampler(t, p, V, 1234)
        o = oracle.Sampler()
        oracle.lib().orc_sampler_init(ctypes.byref(o), t, p, V, 1234)
        tok = 1
        seq = []
        for pos in range(n):
            nxt = a.step_sample(tok, pos, s)
            lg = b.step(tok, pos)
            want = oracle.lib().orc_sample(ctypes.byref(o), lg.ctypes.data)
            assert nxt == want and s.rng == o.rng, "position %d" % pos
            seq.append(nxt)
            tok = nxt
        say("  %d tokens: %s ..." % (n, seq[:12]))
        bad = M.sampler(t, p, V + 1, 1)
        with pytest.raises(RuntimeError, match="vocabulary"):
            a.step_sample(0, 0, bad)
    finally:
        a.close()
        b.close()


def _chain_cases():
    """Vectors for the running sums: (name, values, thresholds)."""
    rng = np.random.default_rng(31)
    out = []
    lg = rng.standard_normal(151936).astype(np.float32) * 3
    e = np.exp((lg - lg.max()) / np.float32(0.8)).astype(np.float32)
    out.append(("exp 151936", e))
    p = np.sort(e / e.sum(dtype=np.float32))[::-1].astype(np.float32)
    out.append(("sorted p", np.ascontiguousarray(p)))
    # every addition a tie at s in [1, 2): u = 2^-23, v = 1.5 u
    out.append(("ties", np.array([1.0] + [1.5 * 2.0 ** -23] * 3000, np.float32)))
    # multiples of a half-ulp at several binades, mixed with exact ulps
    k = rng.integers(0, 8, 20000)
    out.append(("half-ulps", np.concatenate([[np.float32(3.0)],
                                             (k * 2.0 ** -23).astype(np.float32)])))
    # powers of two landing exactly on binade edges, zeros, subnormals
    edge = np.array([0.0, 1e-45, 2e-45, 2.0 ** -126, 2.0 ** -125, 0.5, 0.5, 1.0, 2.0, 4.0,
                     2.0 ** 24, 1.0, 1.0, 3.0, 2.0 ** 30, 0.0], np.float32)
    out.append(("edges", np.tile(edge, 700)))
    tiny = (rng.integers(0, 5000, 30000) * 2.0 ** -149).astype(np.float32)
    out.append(("subnormals", tiny))
    wide = (10.0 ** rng.uniform(-40, 30, 50000)).astype(np.float32)
    out.append(("wide range", wide))
    for n in (0, 1, 7, 8191, 8192, 8193, 16385):
        out.append(("n=%d" % n, rng.random(n).astype(np.float32)))
    x = rng.random(30000).astype(np.float32)
    x[12345] = np.inf
    out.append(("inf", x.copy()))
    x[20000] = np.nan
    out.append(("inf then nan", x.copy()))
    y = rng.random(30000).astype(np.float32)
    y[100] = np.nan
    out.append(("nan", y))
    z = rng.random(30000).astype(np.float32)
    z[9000] = -5.0
    out.append(("negative", z))
    return out


def test_chain_sums_bit_equal(gpu):
    """mhip_chain_f32 (the sampler's running sums, computed 8192 additions at
    a time within a binade) against the sequential fp32 loop (numpy's
    float32 accumulate adds in index order): the final sum, and the stop
    index and value of the >= and > searches, bit-equal, on exponentials,
    sorted probabilities, all-tie and half-ulp sequences, binade edges,
    subnormals, a 70-decade range, ragged lengths, and inf / NaN / negative
    values."""
    say("test_chain_sums_bit_equal")
    d_out = gpu.malloc(8)
    cases = _chain_cases()
    # the values go up through one pinned staging buffer
    cap = max(v.nbytes for _, v in cases) + 16
    h_stage = M.lib().mhip_host_malloc(gpu.h, cap)
    assert h_stage, M.lib().mhip_error(gpu.h).decode()
    stage = np.ctypeslib.as_array(ctypes.cast(h_stage, ctypes.POINTER(ctypes.c_float)), (cap // 4,))
    for name, v in cases:
        n = v.size
        d_v = gpu.malloc(16 * ((n + 3) // 4) + 16)  # n rounded up to 4 values, and more
        if n:
            stage[:n] = v
            gpu.check(M.lib().mhip_h2d(gpu.h, d_v, h_stage, v.nbytes), "h2d")
        with np.errstate(invalid="ignore", over="ignore"):
            c = np.add.accumulate(v, dtype=np.float32) if n else np.zeros(0, np.float32)
        total = c[-1] if n else np.float32(0.0)
        fin = c[np.isfinite(c)]
        thrs = [np.float32(0.5)] + ([fin[len(fin) // 3], fin[-1], np.float32(fin[-1] * 2)]
                                    if fin.size else [])
        runs = [(M.MHIP_CHAIN_SUM, np.float32(0.0))]
        runs += [(m, t) for t in thrs for m in (M.MHIP_CHAIN_GE, M.MHIP_CHAIN_GT)]
        for mode, thr in runs:
            gpu.check(M.lib().mhip_chain_f32(gpu.h, d_v, n, mode, float(thr), d_out), name)
            got = gpu.download(d_out, (2,), np.int32)
            if mode == M.MHIP_CHAIN_SUM:
                k, val = n, total
            else:
                with np.errstate(invalid="ignore"):
                    hit = c >= thr if mode == M.MHIP_CHAIN_GE else thr < c
                k = int(np.argmax(hit)) if hit.any() else n
                val = c[k] if k < n else total
            gv = np.array([got[0]], np.int32).view(np.float32)[0]
            assert got[1] == k, (name, mode, float(thr), int(got[1]), k)
            assert np.array([gv]).view(np.uint32)[0] == np.array([val], np.float32).view(np.uint32)[0], \
                (name, mode, float(thr), float(gv), float(val))
        gpu.free(d_v)
        say("  %-14s n=%-6d sum %r and %d searches bit-equal" % (name, n, float(total), len(runs) - 1))
    gpu.free(d_out)
    M.lib().mhip_host_free(gpu.h, h_stage)
