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
